"""GPU parity across the forward's kernel routes near their boundaries.

fmx_fwd picks, for single queries, the streaming kernel with one or two docs
per workgroup or the tiled kernel by query rows, doc length and width, and
pairs per-query docs. This file draws seeded shapes on both sides of those
boundaries (query rows 32/33, 64/65, 128/129; doc lengths 96/97, 160/161,
256/257, 512/513; widths 64, 96, 128, 256) with ragged lengths, empty docs and
odd doc counts, and checks every score against the float64 oracle (1e-2
absolute, the fp16 bar).
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


@pytest.mark.parametrize("Lq, Ld, d, B, tiled", [
    (64, 77, 128, 9, False),     # 64 rows: streamed
    (65, 77, 128, 9, True),      # 65 rows over short docs: tiled
    (128, 128, 128, 7, True),
    (128, 129, 128, 7, False),   # 65-128 rows over longer docs: streamed
    (129, 300, 128, 6, True),    # several streaming passes over mid-length docs: tiled
    (129, 513, 128, 5, False),
    (100, 96, 120, 8, True),     # masked width
    (300, 64, 100, 5, True),     # partial 8-wide chunk, queries straddling row blocks
    (128, 77, 256, 6, True),     # d = 256 over short docs
    (129, 300, 256, 5, False),   # d = 256 over longer docs: streamed (split into passes)
])
def test_int8_tiled_routes(oracle_mod, Lq, Ld, d, B, tiled):
    """uint8 docs take the tiled kernel from 65 query rows over docs of up to
    128 tokens, and from 129 rows over up to 512 at d <= 128. There each code
    is dequantised to fp16 before the MFMA, so besides the oracle check the
    scores must equal, bit for bit, the fp16 path's on the fp16-dequantised
    docs wherever that path also runs tiled (d <= 128)."""
    from oracle import oracle_np

    seed = 1300 + Lq + Ld + d
    Q = sim((Lq, d), seed)
    x = sim((B, Ld, d), seed + 1, torch.float32)
    codes, s, m = fm.quantize_int8(x)
    lengths = torch.randint(0, Ld + 2, (B,), generator=torch.Generator().manual_seed(seed), dtype=torch.int32)
    lengths[0] = Ld
    lengths[2] = 0
    out = fm.flash_maxsim_int8(Q.to(DEV), codes.to(DEV), s.to(DEV), m.to(DEV), lengths.to(DEV))
    _check(out, oracle_mod.maxsim_int8(to_np32(Q), codes.numpy(), to_np32(s), to_np32(m), lengths.numpy()))
    dq = torch.from_numpy(oracle_np.dequantize_fp16_np(codes.numpy(), s.numpy(), m.numpy()))
    if tiled and d <= 128:
        ref16 = fm.flash_maxsim(Q.to(DEV), dq.to(DEV), lengths.to(DEV))
        assert torch.equal(out, ref16)
    _check(out, oracle_mod.maxsim(to_np32(Q), dq.float().numpy(), lengths.numpy())[0])


@pytest.mark.parametrize("Lq, Ld, d, B", [
    (32, 301, 128, 7),    # stream, 16-byte code rows, scale rows 2-byte aligned
    (32, 77, 96, 9),      # stream, two-tile ring
    (128, 301, 512, 5),   # split-d, 16-byte code rows
    (32, 77, 384, 6),
    (32, 75, 1000, 4),    # split-d, 8-byte code rows (no 16-byte loads)
    (100, 77, 128, 6),    # tiled kernel (65+ query rows over docs of up to 128 tokens)
    (96, 301, 128, 5),    # stream, eight query blocks: fp16 dequantisation of each tile
])
def test_int8_unaligned_scale_rows_routes(oracle_mod, Lq, Ld, d, B):
    """Scale and min rows that start anywhere on a 2-byte boundary: views one
    element into a wider store (read in place, NaN in the column before), so
    doc b's first scale sits 2 bytes past a 4-byte boundary for some docs and
    on one for others. The kernels read them with aligned 12-byte loads and
    byte shifts, and keep 16-byte code loads where the code rows allow."""
    seed = 1400 + Ld + d
    Q = sim((Lq, d), seed)
    x = sim((B, Ld, d), seed + 1, torch.float32)
    codes, s, m = fm.quantize_int8(x)
    lengths = torch.randint(0, Ld + 2, (B,), generator=torch.Generator().manual_seed(seed), dtype=torch.int32)
    lengths[0] = Ld
    lengths[1] = Ld - 1
    s_store = torch.full((B, Ld + 1), float("nan"), dtype=torch.float16, device=DEV)
    m_store = torch.full((B, Ld + 1), float("nan"), dtype=torch.float16, device=DEV)
    s_store[:, 1:] = s[..., 0].to(DEV)
    m_store[:, 1:] = m[..., 0].to(DEV)
    out = fm.flash_maxsim_int8(Q.to(DEV), codes.to(DEV), s_store[:, 1:], m_store[:, 1:], lengths.to(DEV))
    _check(out, oracle_mod.maxsim_int8(to_np32(Q), codes.numpy(), to_np32(s), to_np32(m), lengths.numpy()))


@pytest.mark.parametrize("Lq, Ld, B", [(96, 300, 6), (128, 200, 5), (64, 150, 7), (80, 512, 4)])
def test_single_query_tiled_train_routes(oracle_mod, Lq, Ld, B):
    """Single queries of 33-64 tokens over docs of up to 160 tokens and of
    65-128 over up to 512 run on the tiled kernel's four-wave blocks; the
    training forward takes its argmax instance there. Scores, the saved
    argmax and both gradients are checked against the oracle."""
    from flash_maxsim_amd.flash_maxsim import _launch_fwd, _prep

    d = 128
    Q = sim((Lq, d), 1500 + Lq + Ld)
    D = sim((B, Ld, d), 1501 + Lq + Ld)
    g = torch.linspace(-1.0, 2.0, B, dtype=torch.float32)
    Qg, Dg = Q.to(DEV).requires_grad_(True), D.to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train(Qg, Dg)
    (s * g.to(DEV)).sum().backward()
    Qn, Dn = to_np32(Q), to_np32(D)
    from test_gpu_parity import assert_argmax

    ref, am_ref, best = oracle_mod.maxsim(Qn, Dn, want_argmax=True)
    _check(s, ref[0])
    _, am = _launch_fwd(_prep(Q.to(DEV), torch.float16)[None], _prep(D.to(DEV), torch.float16), None, 1, B, Lq, Ld, d,
                        True, True)
    assert_argmax(am, am_ref, best, Qn, Dn, d)
    dQ_ref, dD_ref = oracle_mod.bwd(Qn, Dn, am.cpu().numpy(), g.numpy())
    np.testing.assert_allclose(Qg.grad.double().cpu().numpy(), dQ_ref, rtol=2e-3, atol=ATOL)
    np.testing.assert_allclose(Dg.grad.double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)


@pytest.mark.parametrize("Lq, Ld, d, dtype", [
    (65, 512, 128, torch.float16),    # 65-128 rows up to 512 tokens: tiled, four-wave 128-row block
    (128, 513, 128, torch.float16),   # past 512 tokens: streamed
    (64, 160, 128, torch.bfloat16),   # 33-64 rows up to 160 tokens: tiled, four-wave 64-row block
    (64, 161, 128, torch.float16),    # past 160 tokens: streamed
    (33, 160, 96, torch.float16),     # masked width
    (128, 512, 96, torch.bfloat16),
    (100, 300, 128, torch.float16),
])
def test_single_query_four_wave_boundaries(oracle_mod, Lq, Ld, d, dtype):
    B = 37
    Q = sim((Lq, d), 1600 + Lq + Ld, dtype)
    D = sim((B, Ld, d), 1601 + Lq + Ld, dtype)
    lengths = torch.randint(0, Ld + 2, (B,), generator=torch.Generator().manual_seed(Lq * Ld), dtype=torch.int32)
    lengths[0], lengths[1] = Ld, 0
    out = fm.flash_maxsim(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    _check(out, oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0])


def test_int8_padding_route_difference_bounded(oracle_mod):
    """The same uint8 docs padded to 128 tokens (tiled kernel: each value
    rounded to fp16 before the dot product) and to 129 (streamed: the affine
    map applied to the fp32 dot product), d = 256, 100 query tokens. Scores
    are not padding-invariant. The 128-token scores must match the oracle on
    the fp16-dequantised docs within Higham's bound of the fp32 sums (so the
    route computes exactly that); the oracle's own fp16-vs-fp32 difference must
    stay within the fp16 rounding bound sum_q max_j sum_k |Q_qk| (2^-11 |x_jk| +
    2^-25); and the two routes' scores must differ by under 1e-3, the figure
    the C header states."""
    from oracle.oracle_np import dequantize_fp16_np, dequantize_np
    from test_gpu_parity import MFMA_MARGIN, gamma

    B, Lq, d = 40, 100, 256
    Q = sim((Lq, d), 1700)
    x = sim((B, 128, d), 1701, torch.float32)
    codes, s, m = fm.quantize_int8(x)
    lengths = torch.randint(1, 129, (B,), generator=torch.Generator().manual_seed(1702), dtype=torch.int32)
    lengths[0] = 128
    c129 = torch.zeros(B, 129, d, dtype=torch.uint8)
    s129 = torch.ones(B, 129, 1, dtype=torch.float16)
    m129 = torch.zeros(B, 129, 1, dtype=torch.float16)
    c129[:, :128], s129[:, :128], m129[:, :128] = codes, s, m
    Qd, ld = Q.to(DEV), lengths.to(DEV)
    out128 = fm.flash_maxsim_int8(Qd, codes.to(DEV), s.to(DEV), m.to(DEV), ld).double().cpu().numpy()
    out129 = fm.flash_maxsim_int8(Qd, c129.to(DEV), s129.to(DEV), m129.to(DEV), ld).double().cpu().numpy()
    Qn, ln = to_np32(Q), lengths.numpy()
    ref32 = oracle_mod.maxsim_int8(Qn, codes.numpy(), to_np32(s), to_np32(m), ln)
    x16 = dequantize_fp16_np(codes.numpy(), s.numpy(), m.numpy()).astype(np.float32)
    ref16, _, best16 = oracle_mod.maxsim(Qn, x16, ln, want_argmax=True)
    ref16 = ref16[0]
    assert np.abs(out128 - ref32).max() <= 1e-2 and np.abs(out129 - ref32).max() <= 1e-2
    qa = np.abs(Qn.astype(np.float64))  # [Lq, d]
    valid = np.arange(128)[None, :, None] < ln[:, None, None]

    def per_score(per):  # [B, 128, Lq] bound per similarity -> [B] bound per score
        return np.where(valid, per, 0.0).max(axis=1).sum(axis=1)

    A16 = np.abs(x16.astype(np.float64)) @ qa.T  # [B, 128, Lq]: sum_k |Q_qk x16_jk|
    # the similarities' bound, plus the fp32 sum of the Lq row maxima
    tiled_bound = per_score(MFMA_MARGIN * gamma(d) * A16) + gamma(Lq) * np.abs(best16).sum(axis=1)
    assert (np.abs(out128 - ref16) <= tiled_bound * 1.001).all()
    A32 = np.abs(dequantize_np(codes.numpy(), s.numpy(), m.numpy()).astype(np.float64)) @ qa.T
    rounding = per_score(2.0**-11 * A32 + 2.0**-25 * qa.sum(1)[None, None, :])
    assert (np.abs(ref16 - ref32) <= rounding * 1.001).all()
    diff = np.abs(out128 - out129)
    print(f"uint8 padding 128 vs 129: max |diff| {diff.max():.3e}; fp16 rounding bound {rounding.min():.3e}")
    assert diff.max() < 1e-3


@pytest.mark.parametrize("Lq, Ld, dst, d, B", [
    (128, 1024, 128, 128, 9),   # 64 tiles per full doc, past the four-tile ring
    (65, 300, 128, 128, 7),
    (100, 132, 96, 96, 11),     # ring start and tail only
    (97, 200, 112, 100, 6),     # d = 100 in rows of 112: a partial 8-wide chunk, codes past d in the row
    (128, 516, 80, 80, 5),
])
def test_int8_shared_tile_route(oracle_mod, Lq, Ld, dst, d, B):
    """Single uint8 queries of 65-128 tokens at d in (64, 128] over padded
    docs with 16-byte code rows, aligned scale rows and Ld > 128: four waves
    share each dequantised doc tile through LDS, and rows past a doc's length
    load its last row again. Ragged lengths (0, 1, 15, 16, 17, a multiple of
    the ring, Ld), a NaN scale in one doc's padding and a NaN min in another's
    first token. Scores must match the oracle on the fp16-dequantised docs
    within Higham's bound of the fp32 sums, the oracle's uint8 scores within
    the fp16 bar, and a NaN only where a valid token carries one."""
    from oracle.oracle_np import dequantize_fp16_np
    from test_gpu_parity import MFMA_MARGIN, gamma

    seed = 1800 + Lq + Ld + d
    Q = sim((Lq, d), seed)
    x = sim((B, Ld, dst), seed + 1, torch.float32)
    codes_st, s, m = fm.quantize_int8(x)  # codes of all dst columns; the view uses the first d
    codes = codes_st[..., :d]
    lengths = torch.randint(1, Ld + 1, (B,), generator=torch.Generator().manual_seed(seed), dtype=torch.int32)
    fixed = [Ld, 0, 1, 15, 16, 17, 64, Ld - 1, 33, 2, 31]
    lengths[:min(B, len(fixed))] = torch.tensor(fixed[:B], dtype=torch.int32)
    s[2, Ld - 1] = float("nan")  # doc 2 (1 token): past its length, never read
    m[B - 1, 0] = float("nan")    # last doc: token 0 is valid
    out = fm.flash_maxsim_int8(Q.to(DEV), codes.to(DEV), s.to(DEV), m.to(DEV), lengths.to(DEV))
    got = out.double().cpu().numpy()
    cn, ln, Qn = codes.contiguous().numpy(), lengths.numpy(), to_np32(Q)
    ref32 = oracle_mod.maxsim_int8(Qn, cn, to_np32(s), to_np32(m), ln)
    _check(out, ref32)
    x16 = dequantize_fp16_np(cn, s.numpy(), m.numpy()).astype(np.float32)
    ref16, _, best16 = oracle_mod.maxsim(Qn, x16, ln, want_argmax=True)
    ref16 = ref16[0]
    fin = np.isfinite(ref16)
    assert np.array_equal(np.isfinite(got), fin) and np.isnan(got[B - 1]) and got[1] == -np.inf
    valid = np.arange(Ld)[None, :, None] < ln[:, None, None]
    A16 = np.nan_to_num(np.abs(x16.astype(np.float64))) @ np.abs(Qn.astype(np.float64)).T  # [B, Ld, Lq]
    per = np.where(valid, MFMA_MARGIN * gamma(d) * A16, 0.0).max(axis=1).sum(axis=1)
    bound = per + gamma(Lq) * np.where(np.isfinite(best16), np.abs(best16), 0.0).sum(axis=1)
    assert (np.abs(got[fin] - ref16[fin]) <= bound[fin] * 1.001).all()
