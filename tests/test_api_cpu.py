"""CPU-side checks of the boundary: the C ABI library and the Python API.

No kernel runs here. The library must load, export every entry point that
include/fmx.h declares (with the arity the ctypes binding uses), and reject
bad arguments with the documented error codes before any launch. The Python
API must raise the reference's AssertionError on bad ranks/shapes and refuse
CPU tensors instead of falling back to a CPU path.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from flash_maxsim_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fmx.h"

FMX_OK, FMX_ERR_INVALID, FMX_ERR_UNSUPPORTED, FMX_ERR_WORKSPACE = 0, -1, -2, -3


def _header_decls():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(fmx_\w+)\s*\(([^)]*)\)\s*;", text):
        args = m.group(2).strip()
        decls[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return decls


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_and_binding_agree(lib):
    decls = _header_decls()
    assert decls, "no declarations parsed from include/fmx.h"
    assert set(decls) == set(_lib.EXPORTED)
    for name, nargs in decls.items():
        assert len(_lib._SIGNATURES[name][1]) == nargs, name


def test_library_exports_every_declared_symbol(lib):
    for name in _header_decls():
        assert hasattr(lib, name), f"libflashmaxsim.so does not export {name}"


def test_version(lib):
    assert lib.fmx_version().decode() == "0.1.0+mi355x"


FAKE = 0x10000  # aligned, never dereferenced: every call below fails validation first


def _fwd(lib, **kw):
    a = dict(dtype=0, Q=FAKE, qn=0, ql=128, D=FAKE, db=300 * 128, dl=128, lengths=None, scores=FAKE,
             sn=0, sb=1, argmax=None, Nq=1, B=10, Lq=32, Ld=300, d=128, shared=1, ws=None, wsb=0)
    a.update(kw)
    return lib.fmx_fwd(a["dtype"], a["Q"], a["qn"], a["ql"], a["D"], a["db"], a["dl"], a["lengths"],
                       a["scores"], a["sn"], a["sb"], a["argmax"], a["Nq"], a["B"], a["Lq"], a["Ld"],
                       a["d"], a["shared"], a["ws"], a["wsb"], None)


@pytest.mark.parametrize("kw, code, text", [
    (dict(dtype=7), FMX_ERR_INVALID, "dtype"),
    (dict(d=65544, ql=65544, dl=65544, db=65544 * 300), FMX_ERR_UNSUPPORTED, "FMX_MAX_D"),
    (dict(d=8192, ql=8192, dl=8192, db=8192 * 300), FMX_ERR_WORKSPACE, "workspace"),  # d > 4096: similarity chunks
    (dict(ql=100), FMX_ERR_INVALID, "Q row stride"),
    (dict(dl=120), FMX_ERR_INVALID, "D row stride"),
    (dict(db=300 * 128 + 4), FMX_ERR_INVALID, "doc stride"),
    (dict(Lq=0), FMX_ERR_INVALID, "invalid sizes"),
    (dict(Q=FAKE + 2), FMX_ERR_INVALID, "aligned"),
    (dict(Q=None), FMX_ERR_INVALID, "non-null"),
    (dict(Lq=1024), FMX_ERR_WORKSPACE, "workspace"),
    (dict(Ld=2**24), FMX_ERR_UNSUPPORTED, "exceeds 2 GiB"),
])
def test_fwd_rejects_bad_arguments(lib, kw, code, text):
    assert _fwd(lib, **kw) == code
    assert text in lib.fmx_last_error().decode()


def test_noalloc_rejects_scratch_overflow(lib):
    # 100 queries of 1024 tokens over 10000 per-query docs: 8 passes of partial
    # sums, 32 MB, beyond the 16 MiB static scratch; refused before any launch.
    need = lib.fmx_fwd_workspace_bytes(100, 10000, 1024, 300, 128)
    assert need == 8 * 100 * 10000 * 4 > (16 << 20)
    rc = lib.fmx_fwd_noalloc(0, FAKE, 1024 * 128, 128, FAKE, 300 * 128, 128, None, FAKE, 10000, 1, None,
                             100, 10000, 1024, 300, 128, 0, None)
    assert rc == FMX_ERR_UNSUPPORTED
    assert "FMX_NOALLOC_SCRATCH_BYTES" in lib.fmx_last_error().decode()


def test_fwd_empty_batch_is_a_no_op(lib):
    assert _fwd(lib, B=0, Q=None, D=None, scores=None) == FMX_OK
    assert lib.fmx_last_error().decode() == ""


def test_workspace_sizes(lib):
    # Lq <= 128 at d <= 256 runs in one pass: no workspace.
    assert lib.fmx_fwd_workspace_bytes(1, 5000, 32, 300, 128) == 0
    assert lib.fmx_fwd_workspace_bytes(100, 5000, 32, 300, 128) == 0
    # Lq = 1024 at d = 128: 8 passes of 128 query tokens.
    assert lib.fmx_fwd_workspace_bytes(1, 10, 1024, 64, 128) == 8 * 10 * 4
    # d = 1024 (split-d): 8 query blocks of 16 per pass -> Lq = 128 in one pass.
    assert lib.fmx_fwd_workspace_bytes(1, 1000, 128, 512, 1024) == 0
    assert lib.fmx_fwd_int8_workspace_bytes(5000, 32, 1024, 128) == 0
    assert lib.fmx_bwd_workspace_bytes(1000, 128, 512, 1024) > 0


def test_fwd_topk_arguments_and_workspace(lib):
    # the scoring part of the workspace is sized for any k, k = 0 included
    ws0 = lib.fmx_fwd_topk_workspace_bytes(10, 1024, 64, 128, 0)
    assert ws0 >= lib.fmx_fwd_workspace_bytes(1, 10, 1024, 64, 128) > 0
    assert lib.fmx_fwd_topk_workspace_bytes(10, 1024, 64, 128, 5) >= ws0
    assert lib.fmx_fwd_topk_workspace_bytes(5000, 32, 300, 128, 100) == 0  # one pass, one chunk

    def call(B, Lq, k, ws, nbytes):
        return lib.fmx_fwd_topk(0, FAKE, 128, FAKE, 300 * 128, 128, None, B, Lq, 300, 128, k, FAKE, FAKE, FAKE,
                                ws, nbytes, None)

    assert call(10, 32, 11, None, 0) == FMX_ERR_INVALID
    assert "exceeds the 10 scores" in lib.fmx_last_error().decode()
    assert call(9000, 32, 8193, None, 0) == FMX_ERR_UNSUPPORTED  # FMX_MAX_TOPK = 8192
    assert call(10, 1024, 3, None, 0) == FMX_ERR_WORKSPACE
    assert call(10, 1024, 3, FAKE + 16, 1 << 20) == FMX_ERR_INVALID
    assert "256-byte aligned" in lib.fmx_last_error().decode()


def test_int8_and_bwd_reject_bad_arguments(lib):
    rc = lib.fmx_fwd_int8(FAKE, 128, FAKE, 300 * 128, 128, FAKE + 1, FAKE, 300, None, FAKE,
                          10, 32, 300, 128, None, 0, None)
    assert rc == FMX_ERR_INVALID and "2-byte aligned" in lib.fmx_last_error().decode()
    rc = lib.fmx_bwd(0, FAKE, 128, FAKE, 300 * 128, 128, FAKE, FAKE, FAKE, None, 10, 32, 300, 128,
                     None, 0, None)
    assert rc == FMX_ERR_WORKSPACE
    rc = lib.fmx_bwd(0, FAKE, 128, FAKE, 300 * 128, 128, FAKE, FAKE, None, None, 10, 32, 300, 128,
                     None, 0, None)
    assert rc == FMX_OK  # nothing requested


def test_bwd_limits(lib):
    # any Nq*Lq: the dD index runs in chunks of 8192 entries (two here)
    assert lib.fmx_bwd_batched_workspace_bytes(70, 6, 128, 64, 128) >= 2 * 6 * 64 * 4 + 6 * 8960 * 2
    # docs of 2^19 tokens or more are refused before any launch
    Ld = 1 << 19
    rc = lib.fmx_bwd_batched(0, FAKE, 0, 8, FAKE, Ld * 8, 8, None, FAKE, FAKE, 0, 1, None, FAKE, 1, 2, 4, Ld, 8,
                             None, 0, None)
    assert rc == FMX_ERR_UNSUPPORTED and "Ld < 2^19" in lib.fmx_last_error().decode()


def test_sparse_rejects_bad_arguments(lib):
    rc = lib.fmx_fwd_sparse(0, FAKE, 128, 32, FAKE, 300 * 128, 128, None, 16, 1, 16, None, FAKE,
                            10, 300, 128, None, 0, None)
    assert rc == FMX_ERR_INVALID and "indices" in lib.fmx_last_error().decode()


def test_quantize_and_packed_reject_bad_arguments(lib):
    rc = lib.fmx_quantize_int8(7, FAKE, 300 * 128, 128, 10, 300, 128, None, None, 0, FAKE, 128, FAKE, FAKE, 300, None)
    assert rc == FMX_ERR_INVALID and "source dtype" in lib.fmx_last_error().decode()
    rc = lib.fmx_quantize_int8(2, FAKE, 300 * 128, 100, 10, 300, 128, None, None, 0, FAKE, 128, FAKE, FAKE, 300, None)
    assert rc == FMX_ERR_INVALID and "row strides" in lib.fmx_last_error().decode()
    rc = lib.fmx_quantize_int8(2, FAKE, 300 * 128, 128, 10, 300, 128, None, None, 0, FAKE, 128, FAKE + 1, FAKE, 300,
                               None)
    assert rc == FMX_ERR_INVALID and "2-byte aligned" in lib.fmx_last_error().decode()
    rc = lib.fmx_quantize_int8(2, FAKE, 300 * 128, 128, 10, 300, 128, FAKE, FAKE, -1, FAKE, 128, FAKE, FAKE, 0, None)
    assert rc == FMX_ERR_INVALID and "tok_rows" in lib.fmx_last_error().decode()
    assert lib.fmx_quantize_int8(2, None, 0, 128, 0, 300, 128, None, None, 0, None, 128, None, None, 300, None) == FMX_OK
    rc = lib.fmx_fwd_packed(0, FAKE, 128, 32, FAKE, 128, 1000, None, FAKE, None, FAKE, 10, 300, 128, None, 0, None)
    assert rc == FMX_ERR_INVALID and "tok_group" in lib.fmx_last_error().decode()
    rc = lib.fmx_fwd_int8_packed(FAKE, 128, 32, FAKE, 128, FAKE, FAKE, 1000, FAKE, None, None, FAKE, 10, 300, 128,
                                 None, 0, None)
    assert rc == FMX_ERR_INVALID and "lengths" in lib.fmx_last_error().decode()
    assert lib.fmx_fwd_packed_workspace_bytes(10, 32, 300, 128) == 0
    # uint8 docs: 128 query tokens per pass at d = 128, so 200 tokens take 2 passes
    assert lib.fmx_fwd_int8_packed_workspace_bytes(10, 200, 300, 128) == 2 * 10 * 4


def test_packed_layout_on_cpu():
    # The packing itself is torch host logic; only scoring needs the GPU.
    import flash_maxsim_amd as fm

    D = torch.arange(6 * 9 * 8, dtype=torch.float32).reshape(6, 9, 8).half()
    lengths = torch.tensor([9, 0, 1, 4, 5, 12])  # 12 clamps to 9
    pk = fm.pack_docs(D, lengths)
    assert pk.lengths.tolist() == [9, 0, 1, 4, 5, 9] and pk.max_len == 9
    assert pk.tok_group.tolist() == [0, 3, 3, 4, 5, 7]  # exclusive prefix sum of ceil(len / 4)
    assert pk.tokens.shape == (40, 8)
    for b, L in enumerate(pk.lengths.tolist()):
        r0 = 4 * pk.tok_group[b].item()
        assert torch.equal(pk.tokens[r0:r0 + L], D[b, :L])
        assert not pk.tokens[r0 + L:r0 + 4 * ((L + 3) // 4)].any()
    full = fm.pack_docs(D)
    assert full.tokens.shape == (6 * 12, 8) and full.lengths.tolist() == [9] * 6


# ---------------------------------------------------------- Python API ----

def test_python_api_asserts_like_the_reference():
    import flash_maxsim_amd as fm

    Q, D = torch.zeros(4, 8), torch.zeros(2, 5, 8)
    with pytest.raises(AssertionError):
        fm.flash_maxsim(Q[None], D)
    with pytest.raises(AssertionError):
        fm.flash_maxsim(Q, D[..., :4])
    with pytest.raises(AssertionError):
        fm.flash_maxsim_batched(Q, D)
    with pytest.raises(AssertionError):
        fm.flash_maxsim_batched(Q[None], D[None], shared_docs=True)
    with pytest.raises(AssertionError):
        fm.flash_maxsim_batched(Q[None].expand(2, 4, 8), D[None], shared_docs=False)
    with pytest.raises(AssertionError):
        fm.flash_maxsim_int8(Q, torch.zeros(2, 5, 8, dtype=torch.uint8)[0], torch.zeros(2, 5), torch.zeros(2, 5))
    with pytest.raises(AssertionError):
        fm.flash_maxsim_sparse(Q, D, torch.zeros(3, 2, dtype=torch.int32))
    with pytest.raises(AssertionError):
        fm.quantize_int8(D[0])


def test_python_api_refuses_cpu_tensors():
    import flash_maxsim_amd as fm

    Q, D = torch.zeros(4, 8, dtype=torch.float16), torch.zeros(2, 5, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fm.flash_maxsim(Q, D)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fm.flash_maxsim_train(Q, D)


def test_operand_prep_reads_abi_layouts_in_place():
    """Views the C ABI accepts (row strides multiple of 8 and >= d, unit stride
    along d, 16-byte aligned, kernel dtype) pass through uncopied, d % 8 != 0
    included; everything else becomes a zero-padded contiguous copy."""
    from flash_maxsim_amd.flash_maxsim import _prep

    f16 = torch.float16
    store = torch.full((6, 40, 104), float("nan"), dtype=f16)
    view = store[1:5, :33, :100]                     # padded store, d = 100
    assert _prep(view, f16) is view
    q = torch.zeros(64, 136, dtype=f16)[::2, :128]   # strided rows
    assert _prep(q, f16) is q
    codes = torch.zeros(4, 40, 112, dtype=torch.uint8)[:, :, :100]  # uint8 codes, no cast
    assert _prep(codes, None) is codes

    for t, dt in [(torch.zeros(3, 10, 100, dtype=f16), f16),            # contiguous, d % 8 != 0
                  (torch.zeros(3, 128, 64, dtype=f16).transpose(1, 2), f16),
                  (store[:, :, 4:100], f16),                            # 8-byte aligned base
                  (store[:, :, :100], torch.bfloat16)]:                 # needs a cast
        out = _prep(t, dt)
        assert out.data_ptr() != t.data_ptr() or out.dtype != t.dtype
        assert out.is_contiguous() and out.shape[-1] % 8 == 0 and out.data_ptr() % 16 == 0
        assert out.dtype == dt
        d = t.shape[-1]
        torch.testing.assert_close(out[..., :d].float(), t.float().to(dt).float(), equal_nan=True)
        assert not out[..., d:].float().any()
    # overlapping rows (row stride 8 < d = 96) are copied, not passed through
    ov = torch.zeros(3 * 10 * 96, dtype=f16).as_strided((3, 10, 96), (960, 8, 1))
    assert _prep(ov, f16).stride(-2) == 96


def test_naive_functions_run_on_cpu():
    import flash_maxsim_amd as fm

    Q = torch.randn(4, 8)
    D = torch.randn(3, 5, 8)
    s = fm.maxsim_naive(Q, D, torch.tensor([5, 2, 0]))
    assert s.shape == (3,) and torch.isinf(s[2]) and s[2] < 0
    codes, sc, mn = fm.quantize_int8(D)
    assert codes.dtype == torch.uint8 and sc.shape == (3, 5, 1) and mn.dtype == torch.float16
    assert fm.dequantize_int8(codes, sc, mn).shape == D.shape
    idx = torch.tensor([[0, 1], [2, 3], [3, 3]])
    assert fm.maxsim_sparse_naive(Q, D, idx).shape == (3,)


def test_dequantize_int8_values():
    """dequantize_int8 (reference flash_maxsim_quant.py:31-33) bit for bit:
    against the NumPy restatement (float32 multiply, then add), against the
    hand-derived quant fixture (codes on exact binary grids decode to the
    original rows); fp16 arithmetic must differ somewhere."""
    from pathlib import Path

    import flash_maxsim_amd as fm
    from oracle.oracle_np import dequantize_np

    g = torch.Generator().manual_seed(5)
    D = torch.nn.functional.normalize(torch.randn(4, 33, 96, generator=g), dim=-1) * 3.0
    codes, sc, mn = fm.quantize_int8(D)
    got = fm.dequantize_int8(codes, sc, mn)
    assert got.dtype == torch.float32 and got.shape == D.shape
    want = dequantize_np(codes.numpy(), sc.numpy(), mn.numpy())
    np.testing.assert_array_equal(got.numpy().view(np.uint32), want.view(np.uint32))
    # (code * step is exact in float32, 8-bit codes times 11-bit fp16 steps, so
    # only the add rounds.) Planted mistake: the same formula in fp16
    # arithmetic, as the reference's uint8 kernel dequantises, must differ.
    half = (codes.numpy().astype(np.float16) * sc.numpy() + mn.numpy()).astype(np.float32)
    assert not np.array_equal(half.view(np.uint32), got.numpy().view(np.uint32))
    f = dict(np.load(Path(__file__).resolve().parent / "golden" / "quant.npz"))
    rows = fm.dequantize_int8(torch.from_numpy(f["codes"]), torch.from_numpy(f["scales"]),
                              torch.from_numpy(f["mins"])).numpy()
    for r in (0, 3):  # exact binary grids: step and min are fp16-exact, codes decode exactly
        np.testing.assert_array_equal(rows[0, r], f["D"][0, r])
    # row 2: step 1/16, min 0, half-way values rounded to even codes: code / 16
    np.testing.assert_array_equal(rows[0, 2], f["codes"][0, 2].astype(np.float32) / 16)
    np.testing.assert_array_equal(rows[0, 1], np.full(f["D"].shape[-1], 0.5, np.float32))  # scale 0 -> min


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libflashmaxsim.so")
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load()


def test_pack_docs_sorted_layout_cpu():
    """pack_docs(sort_by_length=True) on the CPU: slots longest first (stable
    among equal lengths), tok_group and lengths per slot, slot s holding the
    rows of doc doc_ids[s] back to back in 4-row groups, zero rows between."""
    import flash_maxsim_amd as fm

    B, Ld, d = 9, 11, 5
    D = torch.arange(B * Ld * d, dtype=torch.float32).reshape(B, Ld, d).half()
    lengths = torch.tensor([3, 11, 0, 7, 7, 1, 11, 4, 2], dtype=torch.int32)
    p = fm.pack_docs(D, lengths, sort_by_length=True)
    ids = p.doc_ids.long()
    assert p.doc_ids.dtype == torch.int32
    assert ids.tolist() == [1, 6, 3, 4, 7, 0, 8, 5, 2]
    assert p.lengths.tolist() == [11, 11, 7, 7, 4, 3, 2, 1, 0]
    groups = (p.lengths.long() + 3) // 4
    assert p.tok_group.tolist() == (torch.cumsum(groups, 0) - groups).tolist()
    assert p.tokens.shape[0] == 4 * int(groups.sum()) and p.max_len == 11
    for s in range(B):
        r0, n = 4 * int(p.tok_group[s]), int(p.lengths[s])
        assert torch.equal(p.tokens[r0:r0 + n], D[ids[s], :n])
        assert torch.all(p.tokens[r0 + n:r0 + 4 * int(groups[s])] == 0)
    plain = fm.pack_docs(D, lengths)
    assert plain.doc_ids is None and plain.lengths.tolist() == lengths.tolist()
