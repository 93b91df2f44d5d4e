"""GPU parity of the HIP uint8 encoder and the packed-doc forwards.

quantize_int8 on a GPU tensor runs libflashmaxsim's encoder; its codes, fp16
scales and fp16 mins must be bit-identical to the CPU oracle's restatement of
the reference formula (oracle/maxsim_oracle.c, itself pinned to torch and to
the golden quantiser fixture). The packed layout must hold exactly those rows,
and the packed forwards must score like the oracle on the padded docs (1e-2,
the north-star bar) and bit-identically to the padded GPU path, which runs the
same kernel arithmetic on the same token rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flash_maxsim_amd as fm
from conftest import ROOT, sim, to_np32

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATOL = 1e-2


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def assert_quant_equal(got, want_codes, want_s, want_m):
    codes, s, m = got
    np.testing.assert_array_equal(codes.cpu().numpy(), want_codes)
    np.testing.assert_array_equal(_bits(s).reshape(-1), np.asarray(want_s).view(np.int16).reshape(-1))
    np.testing.assert_array_equal(_bits(m).reshape(-1), np.asarray(want_m).view(np.int16).reshape(-1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [128, 100, 7, 1024, 2048])
def test_quantize_matches_oracle_bitwise(oracle_mod, dtype, d):
    x = torch.randn(6, 37, d, generator=torch.Generator().manual_seed(d), dtype=torch.float32)
    x[0, 0] = 0.25        # constant row: step floor 1e-8, which fp16 rounds to 0
    x[1, 2, : d // 2] = -1.5
    x = x.to(dtype)
    want = oracle_mod.quantize_int8(to_np32(x))[:3]
    got = fm.quantize_int8(x.to(DEV))
    assert_quant_equal(got, *want)
    # and the torch formula on the CPU (the reference's own code path)
    t_codes, t_s, t_m = fm.quantize_int8(x)
    np.testing.assert_array_equal(got[0].cpu().numpy(), t_codes.numpy())
    np.testing.assert_array_equal(_bits(got[1]), _bits(t_s))


def near_half_rows(seed, nrows, d):
    """fp32 rows whose quotients (x - min) / scale fall on half-integers or
    within 3 ulps of one: each row holds its min and max, then values at
    min + (k + 0.5) * scale (scale as the formula computes it) nudged by -3..3
    ulps, where rounding the product with the reciprocal could pick a different
    code than rounding the correctly rounded quotient."""
    rng = np.random.default_rng(seed)
    out = np.empty((nrows, d), np.float32)
    for r in range(nrows):
        lo = np.float32(rng.standard_normal() * 0.1)
        hi = np.float32(lo + np.float32(abs(rng.standard_normal()) + 0.05))
        step = np.float32(np.float32(hi - lo) / np.float32(255.0))
        k = rng.integers(0, 255, d - 2).astype(np.float32)
        x = (lo + (k + np.float32(0.5)) * step).astype(np.float32)
        x = (x.view(np.int32) + rng.integers(-3, 4, d - 2).astype(np.int32)).view(np.float32)
        out[r, 0], out[r, 1], out[r, 2:] = lo, hi, np.clip(x, lo, hi)
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_quantize_quotients_near_half_integers(oracle_mod, dtype):
    """Codes of values whose quotients sit on or next to half-integers equal the
    oracle's (correctly rounded quotient, then round half to even) bit for bit."""
    x = torch.from_numpy(near_half_rows(11, 16 * 128, 128)).reshape(16, 128, 128).to(dtype)
    want = oracle_mod.quantize_int8(to_np32(x))[:3]
    assert_quant_equal(fm.quantize_int8(x.to(DEV)), *want)


def test_quantize_golden_fixture():
    f = np.load(ROOT / "tests" / "golden" / "quant.npz")
    got = fm.quantize_int8(torch.from_numpy(f["D"]).to(DEV))
    assert_quant_equal(got, f["codes"], f["scales"], f["mins"])


def test_quantize_strided_source(oracle_mod):
    x = torch.randn(4, 50, 160, generator=torch.Generator().manual_seed(5)).half()
    xs = x[:, ::2, 4:132]  # strided rows starting 8 bytes into the row: scalar path
    want = oracle_mod.quantize_int8(to_np32(xs))[:3]
    assert_quant_equal(fm.quantize_int8(xs.to(DEV)), *want)
    assert_quant_equal(fm.quantize_int8(x.to(DEV)[:, ::2, 4:132]), *want)
    assert_quant_equal(fm.quantize_int8(x.to(DEV)[:, ::2, 16:144]), *oracle_mod.quantize_int8(
        to_np32(x[:, ::2, 16:144]))[:3])  # 16-byte aligned rows: vector path


@pytest.mark.parametrize("d", [128, 96, 1024])
def test_quantize_packed_layout(oracle_mod, d):
    B, Ld = 9, 70
    x = sim((B, Ld, d), 40 + d, torch.float32)
    lengths = torch.tensor([70, 0, 1, 3, 4, 5, 69, 35, 80], dtype=torch.int32)  # 80 clamps to 70
    packed = fm.quantize_int8_packed(x.to(DEV), lengths.to(DEV))
    c_ref, s_ref, m_ref, _ = oracle_mod.quantize_int8(to_np32(x))
    tg = packed.tok_group.cpu().numpy()
    L = packed.lengths.cpu().numpy()
    np.testing.assert_array_equal(L, np.clip(lengths.numpy(), 0, Ld))
    groups = (L.astype(np.int64) + 3) // 4
    np.testing.assert_array_equal(tg, np.cumsum(groups) - groups)
    assert packed.codes.shape == (4 * groups.sum(), d) and packed.max_len == 70
    codes = packed.codes.cpu().numpy()
    sb, mb = _bits(packed.scales), _bits(packed.mins)
    for b in range(B):
        r0 = 4 * tg[b]
        np.testing.assert_array_equal(codes[r0:r0 + L[b]], c_ref[b, :L[b]])
        np.testing.assert_array_equal(sb[r0:r0 + L[b]], s_ref[b, :L[b], 0].view(np.int16))
        np.testing.assert_array_equal(mb[r0:r0 + L[b]], m_ref[b, :L[b], 0].view(np.int16))
        pad = slice(r0 + L[b], r0 + 4 * groups[b])
        assert not codes[pad].any() and not sb[pad].any() and not mb[pad].any()


@pytest.mark.parametrize("Lq, d", [(32, 128), (7, 64), (200, 128), (32, 100), (16, 512), (100, 128)])
def test_int8_packed_scores(oracle_mod, Lq, d):
    B, Ld = 40, 90
    Q = sim((Lq, d), 60 + Lq)
    x = sim((B, Ld, d), 61 + d, torch.float32)
    lengths = torch.randint(0, Ld + 1, (B,), generator=torch.Generator().manual_seed(d), dtype=torch.int32)
    lengths[:3] = torch.tensor([0, 1, Ld], dtype=torch.int32)
    packed = fm.quantize_int8_packed(x.to(DEV), lengths.to(DEV))
    out = fm.flash_maxsim_int8_packed(Q.to(DEV), packed)
    codes, s16, m16, _ = oracle_mod.quantize_int8(to_np32(x))
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes, s16.astype(np.float32), m16.astype(np.float32), lengths.numpy())
    got = out.double().cpu().numpy()
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    assert np.abs(got[fin] - ref[fin]).max() <= ATOL
    # same kernel arithmetic as the padded layout
    padded = fm.flash_maxsim_int8(Q.to(DEV), torch.from_numpy(codes).to(DEV), torch.from_numpy(s16).to(DEV),
                                  torch.from_numpy(m16).to(DEV), lengths.to(DEV))
    np.testing.assert_array_equal(out.cpu().numpy(), padded.cpu().numpy())


def test_int8_packed_groups_in_any_order():
    # The contract allows token groups anywhere in [0, T): store the docs of a
    # packed layout in reverse order (with a gap) and expect identical scores.
    B, Ld, d, Lq = 37, 70, 128, 32
    Q = sim((Lq, d), 71)
    x = sim((B, Ld, d), 72, torch.float32)
    lengths = torch.randint(0, Ld + 1, (B,), generator=torch.Generator().manual_seed(5), dtype=torch.int32)
    lengths[:2] = torch.tensor([0, Ld], dtype=torch.int32)
    packed = fm.quantize_int8_packed(x.to(DEV), lengths.to(DEV))
    want = fm.flash_maxsim_int8_packed(Q.to(DEV), packed)
    tg = packed.tok_group.cpu()
    groups = (packed.lengths.cpu().to(torch.int64) + 3) // 4
    total = int(groups.sum()) + 5  # five spare groups at the front
    new_tg = torch.empty_like(tg)
    codes = torch.zeros(4 * total, d, dtype=torch.uint8, device=DEV)
    scales = torch.zeros(4 * total, dtype=torch.float16, device=DEV)
    mins = torch.zeros(4 * total, dtype=torch.float16, device=DEV)
    at = total
    for b in range(B):  # doc 0 last in memory, doc B-1 first
        at -= int(groups[b])
        new_tg[b] = at
        src, dst, n = 4 * int(tg[b]), 4 * at, 4 * int(groups[b])
        codes[dst:dst + n] = packed.codes[src:src + n]
        scales[dst:dst + n] = packed.scales[src:src + n]
        mins[dst:dst + n] = packed.mins[src:src + n]
    moved = fm.PackedInt8Docs(codes, scales, mins, new_tg.to(DEV), packed.lengths, packed.max_len)
    got = fm.flash_maxsim_int8_packed(Q.to(DEV), moved)
    np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())


@pytest.mark.parametrize("cut", [0.3, 0.77])
def test_int8_packed_docs_cut_by_tok_rows(oracle_mod, cut):
    """Token rows at or past tok_rows read as zeros (codes, scales and mins),
    so a doc's tokens there score 0: docs wholly past the end, docs that
    straddle it, in both members of the two-doc workgroups."""
    B, Ld, d, Lq = 41, 70, 128, 32
    Q = sim((Lq, d), 75)
    x = sim((B, Ld, d), 76, torch.float32)
    lengths = torch.randint(1, Ld + 1, (B,), generator=torch.Generator().manual_seed(9), dtype=torch.int32)
    packed = fm.quantize_int8_packed(x.to(DEV), lengths.to(DEV))
    T = int(cut * packed.codes.shape[0])
    cut_docs = fm.PackedInt8Docs(packed.codes[:T], packed.scales[:T], packed.mins[:T], packed.tok_group,
                                 packed.lengths, packed.max_len)
    got = fm.flash_maxsim_int8_packed(Q.to(DEV), cut_docs).double().cpu().numpy()
    codes, s16, m16, _ = oracle_mod.quantize_int8(to_np32(x))
    s32, m32 = s16.astype(np.float32).reshape(B, Ld), m16.astype(np.float32).reshape(B, Ld)
    tg = packed.tok_group.cpu().numpy()
    rows = 4 * tg[:, None] + np.arange(Ld)[None, :]
    gone = rows >= T
    assert gone.any(axis=1).sum() >= 2 and (~gone).any(axis=1).sum() >= 2
    codes[gone], s32[gone], m32[gone] = 0, 0.0, 0.0
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes, s32, m32, lengths.numpy())
    assert np.abs(got - ref).max() <= ATOL


@pytest.mark.parametrize("Lq, d, dtype", [(32, 128, torch.float16), (300, 128, torch.float16), (100, 128, torch.float16),
                                          (32, 1024, torch.float16), (20, 96, torch.bfloat16)])
def test_packed_scores(oracle_mod, Lq, d, dtype):
    B, Ld = 30, 80
    Q = sim((Lq, d), 70 + Lq, dtype)
    D = sim((B, Ld, d), 71 + d, dtype)
    lengths = torch.randint(0, Ld + 1, (B,), generator=torch.Generator().manual_seed(Lq), dtype=torch.int32)
    lengths[0] = 0
    packed = fm.pack_docs(D.to(DEV), lengths.to(DEV))
    out = fm.flash_maxsim_packed(Q.to(DEV), packed)
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0]
    got = out.double().cpu().numpy()
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    assert np.abs(got[fin] - ref[fin]).max() <= ATOL
    padded = fm.flash_maxsim(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    np.testing.assert_array_equal(out.cpu().numpy(), padded.cpu().numpy())


def test_packed_four_wave_tiled(oracle_mod):
    # 400-token query over 1600 packed docs: the tiled plan (256 CUs) picks two
    # 256-row blocks of four-wave workgroups, three per CU.
    B, Ld, Lq, d = 1600, 40, 400, 128
    Q = sim((Lq, d), 90)
    D = sim((B, Ld, d), 91)
    lengths = torch.randint(0, Ld + 1, (B,), generator=torch.Generator().manual_seed(92), dtype=torch.int32)
    packed = fm.pack_docs(D.to(DEV), lengths.to(DEV))
    out = fm.flash_maxsim_packed(Q.to(DEV), packed)
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0]
    got = out.double().cpu().numpy()
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    assert np.abs(got[fin] - ref[fin]).max() <= ATOL
    padded = fm.flash_maxsim(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    np.testing.assert_array_equal(out.cpu().numpy(), padded.cpu().numpy())


def test_packed_empty_and_all_empty(oracle_mod):
    Q = sim((32, 128), 80)
    D = sim((5, 16, 128), 81)
    packed = fm.pack_docs(D.to(DEV), torch.zeros(5, dtype=torch.int32, device=DEV))
    assert packed.tokens.shape[0] == 0
    out = fm.flash_maxsim_packed(Q.to(DEV), packed)
    assert torch.isneginf(out).all()
    x = sim((3, 16, 128), 82, torch.float32)
    pk = fm.quantize_int8_packed(x.to(DEV), torch.zeros(3, dtype=torch.int32))
    assert torch.isneginf(fm.flash_maxsim_int8_packed(Q.to(DEV), pk)).all()


def test_quantize_packed_respects_tok_rows(oracle_mod):
    """Rows at or past tok_rows are never written: the buffer has room past T
    filled with a sentinel, which must survive."""
    from flash_maxsim_amd import _lib

    B, Ld, d = 4, 20, 128
    x = sim((B, Ld, d), 90, torch.float32).to(DEV)
    lengths = torch.full((B,), Ld, dtype=torch.int32, device=DEV)
    tg = torch.tensor([0, 5, 10, 15], dtype=torch.int64, device=DEV)  # 80 rows of output
    T = 50
    codes = torch.full((80, d), 7, dtype=torch.uint8, device=DEV)
    scales = torch.full((80,), 7.0, dtype=torch.float16, device=DEV)
    mins = torch.full((80,), 7.0, dtype=torch.float16, device=DEV)
    lib = _lib.load()
    rc = lib.fmx_quantize_int8(_lib.FMX_DTYPE_F32, x.data_ptr(), x.stride(0), x.stride(1), B, Ld, d,
                               lengths.data_ptr(), tg.data_ptr(), T, codes.data_ptr(), d, scales.data_ptr(),
                               mins.data_ptr(), 0, _lib.stream_of(x))
    _lib.check(rc)
    torch.cuda.synchronize()
    assert (codes[T:] == 7).all() and (scales[T:] == 7).all() and (mins[T:] == 7).all()
    c_ref = oracle_mod.quantize_int8(to_np32(x))[0]
    got = codes.cpu().numpy()
    for b in range(B):
        r0 = 4 * int(tg[b])
        n = max(0, min(Ld, T - r0))
        np.testing.assert_array_equal(got[r0:r0 + n], c_ref[b, :n])


@pytest.mark.parametrize(
    "kind, Lq, Ld, d",
    [("f16", 32, 90, 128), ("f16", 32, 40, 128), ("f16", 300, 80, 128), ("f16", 100, 80, 128),
     ("f16", 32, 80, 1024), ("f16", 8, 20, 4100), ("u8", 32, 90, 128), ("u8", 200, 90, 128),
     ("u8", 100, 77, 128), ("u8", 16, 90, 512)],
)
def test_packed_sorted_by_length_same_scores(kind, Lq, Ld, d):
    """Docs laid out longest first (sort_by_length): every kernel route writes
    slot s's score to doc doc_ids[s], so the scores equal the unsorted layout's
    bit for bit (the same rows through the same arithmetic)."""
    B = 300
    gen = torch.Generator().manual_seed(1900 + Lq + d)
    Q = sim((Lq, d), 1901 + d)
    x = sim((B, Ld, d), 1902 + Lq, torch.float32 if kind == "u8" else torch.float16)
    lengths = torch.randint(0, Ld + 1, (B,), generator=gen, dtype=torch.int32)
    lengths[:4] = torch.tensor([0, Ld, 1, 0], dtype=torch.int32)
    if kind == "u8":
        plain = fm.quantize_int8_packed(x.to(DEV), lengths.to(DEV))
        srt = fm.quantize_int8_packed(x.to(DEV), lengths.to(DEV), sort_by_length=True)
        want = fm.flash_maxsim_int8_packed(Q.to(DEV), plain)
        got = fm.flash_maxsim_int8_packed(Q.to(DEV), srt)
        rows_plain, rows_srt = plain.codes, srt.codes
    else:
        plain = fm.pack_docs(x.to(DEV), lengths.to(DEV))
        srt = fm.pack_docs(x.to(DEV), lengths.to(DEV), sort_by_length=True)
        want = fm.flash_maxsim_packed(Q.to(DEV), plain)
        got = fm.flash_maxsim_packed(Q.to(DEV), srt)
        rows_plain, rows_srt = plain.tokens, srt.tokens
    assert plain.doc_ids is None and srt.doc_ids is not None
    ids = srt.doc_ids.long().cpu()
    assert torch.equal(torch.sort(ids).values, torch.arange(B))
    assert torch.all(srt.lengths[:-1] >= srt.lengths[1:])
    assert torch.equal(srt.lengths.cpu(), lengths[ids])
    for s in (0, 1, B // 2, B - 1):  # slot s holds doc ids[s]'s rows
        b, n = int(ids[s]), int(lengths[ids[s]])
        a0, p0 = 4 * int(srt.tok_group[s]), 4 * int(plain.tok_group[b])
        assert torch.equal(rows_srt[a0:a0 + n], rows_plain[p0:p0 + n])
    np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())


def test_packed_doc_ids_out_of_range_not_written():
    """fmx_fwd_packed with doc_ids holding ids outside [0, B): those slots'
    scores are not written (the columns of the docs they displaced keep what
    the caller put there), every other doc's score lands in its column."""
    from flash_maxsim_amd import _lib

    B, Ld, d, Lq = 64, 50, 128, 32
    Q = sim((Lq, d), 1910).to(DEV)
    D = sim((B, Ld, d), 1911).to(DEV)
    lengths = torch.randint(1, Ld + 1, (B,), generator=torch.Generator().manual_seed(1912), dtype=torch.int32)
    packed = fm.pack_docs(D, lengths.to(DEV), sort_by_length=True)
    want = fm.flash_maxsim_packed(Q, packed)
    ids = packed.doc_ids.clone()
    lost = [int(ids[3]), int(ids[40])]
    ids[3], ids[40] = B, -7
    scores = torch.full((B,), 7.0, dtype=torch.float32, device=DEV)
    lib = _lib.load()
    rc = lib.fmx_fwd_packed(
        _lib.dtype_code(Q), Q.data_ptr(), Q.stride(0), Lq, packed.tokens.data_ptr(), packed.tokens.stride(0),
        packed.tokens.shape[0], packed.tok_group.data_ptr(), packed.lengths.data_ptr(), ids.data_ptr(),
        scores.data_ptr(), B, packed.max_len, d, None, 0, torch.cuda.current_stream().cuda_stream,
    )
    _lib.check(rc)
    keep = torch.ones(B, dtype=torch.bool)
    keep[lost] = False
    assert torch.all(scores.cpu()[~keep] == 7.0)
    assert torch.equal(scores.cpu()[keep], want.cpu()[keep])


@pytest.mark.parametrize("d", [128, 100, 16, 8, 7, 1])
def test_quantize_fp16_special_values_bitwise(d):
    """fp16 sources take the packed path (row min/max on pairs of halves, x - min
    formed from each half by a mixed-precision fma): rows with fp16 subnormals,
    +-65504, values one ulp apart and the extremes in either half of a word or
    in a partial last chunk must quantise bit for bit as the reference's torch
    formula does on the CPU."""
    gen = torch.Generator().manual_seed(2200 + d)
    rows = 64
    x = (torch.randn(rows, d, generator=gen) * 4).to(torch.float16)
    tiny = torch.tensor([2.0**-24, 3 * 2.0**-24, 2.0**-14, -(2.0**-24), -1023 * 2.0**-24]).to(torch.float16)
    for r in range(rows):
        k = r % d
        if r % 4 == 0:
            x[r] = tiny[torch.randint(0, len(tiny), (d,), generator=gen)]
        elif r % 4 == 1:
            x[r, k] = 65504.0 if r % 8 == 1 else -65504.0
        elif r % 4 == 2:
            base = x[r, 0].view(torch.int16)
            x[r] = (base + torch.randint(-2, 3, (d,), generator=gen, dtype=torch.int16)).view(torch.float16)
        else:
            x[r, k] = x[r].float().max().half() * 2 + 1  # the maximum at a rotating position
    x3 = x.reshape(8, 8, d)
    got = fm.quantize_int8(x3.to(DEV))
    want = fm.quantize_int8(x3)  # torch formula on the CPU
    np.testing.assert_array_equal(got[0].cpu().numpy(), want[0].numpy())
    np.testing.assert_array_equal(_bits(got[1]), _bits(want[1]))
    np.testing.assert_array_equal(_bits(got[2]), _bits(want[2]))
