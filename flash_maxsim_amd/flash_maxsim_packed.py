"""Packed variable-length docs: no padding in storage or in the scan.

The reference stores docs padded to [B, Ld, d] (fp16, or uint8 codes from
quantize_int8, flash_maxsim/flash_maxsim_quant.py:11-28) and masks the padding
in its kernels (flash_maxsim.py:119-121). Here a collection of docs can instead
be packed: the valid tokens of all docs back to back, doc b starting at token
row 4 * tok_group[b] (token groups of 4 keep every doc's scale rows 8-byte
aligned for the uint8 kernel), with its length in lengths[b]. Scores are the
same as flash_maxsim / flash_maxsim_int8 on the padded docs with
doc_lengths = lengths; storage is sum(ceil(len / 4) * 4) token rows instead of
B * Ld.

This layout has no counterpart in the reference; it is the packed format of
the storage step in front of the scoring path.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import _lib
from .flash_maxsim import _check_devices, _device_guard, _kernel_dtype, _prep
from .flash_maxsim_quant import _SRC_CODES, _quant_source


class PackedDocs(NamedTuple):
    """fp16/bf16 docs packed by pack_docs."""

    tokens: torch.Tensor     # [T, d] token rows of every doc
    tok_group: torch.Tensor  # [B] int64: doc b starts at row 4 * tok_group[b]
    lengths: torch.Tensor    # [B] int32 valid tokens per doc
    max_len: int             # max(lengths), the Ld of the padded equivalent


class PackedInt8Docs(NamedTuple):
    """uint8 docs packed by quantize_int8_packed."""

    codes: torch.Tensor      # [T, d] uint8
    scales: torch.Tensor     # [T] fp16 per-token step
    mins: torch.Tensor       # [T] fp16 per-token minimum
    tok_group: torch.Tensor  # [B] int64
    lengths: torch.Tensor    # [B] int32
    max_len: int


def _layout(B: int, Ld: int, doc_lengths, device) -> tuple[torch.Tensor, torch.Tensor, int, int]:
    """(lengths int32 clamped to [0, Ld], tok_group int64, total rows T, max_len)."""
    if doc_lengths is None:
        lengths = torch.full((B,), Ld, dtype=torch.int32, device=device)
    else:
        assert doc_lengths.numel() == B, f"doc_lengths has {doc_lengths.numel()} entries, expected {B}"
        lengths = doc_lengths.to(device=device, dtype=torch.int32).reshape(B).clamp(0, Ld).contiguous()
    groups = (lengths.to(torch.int64) + 3) // 4
    ends = torch.cumsum(groups, 0)
    tok_group = (ends - groups).contiguous()
    T = 4 * int(ends[-1]) if B > 0 else 0
    max_len = int(lengths.max()) if B > 0 else 0
    return lengths, tok_group, T, max_len


def pack_docs(D: torch.Tensor, doc_lengths=None) -> PackedDocs:
    """Packs the first doc_lengths[b] tokens of each doc of D [B, Ld, d]
    (all Ld when doc_lengths is None; lengths are clamped to [0, Ld]).
    Rows between a doc's length and its next 4-token boundary are zero."""
    assert D.dim() == 3
    B, Ld, d = D.shape
    lengths, tok_group, T, max_len = _layout(B, Ld, doc_lengths, D.device)
    tokens = torch.zeros(T, d, dtype=D.dtype, device=D.device)
    if T:
        j = torch.arange(Ld, device=D.device)
        valid = j[None, :] < lengths[:, None].to(torch.int64)
        rows = (4 * tok_group[:, None] + j[None, :])[valid]
        tokens[rows] = D[valid]
    return PackedDocs(tokens, tok_group, lengths, max_len)


def quantize_int8_packed(D: torch.Tensor, doc_lengths=None) -> PackedInt8Docs:
    """quantize_int8 of the first doc_lengths[b] tokens of each doc of D
    [B, Ld, d] (on the GPU), written straight into the packed layout by one
    pass of the HIP encoder: per token the codes, scale and min are bit-equal
    to quantize_int8(D)'s."""
    assert D.dim() == 3
    B, Ld, d = D.shape
    src = _quant_source(D)
    dev = _check_devices(src)
    lengths, tok_group, T, max_len = _layout(B, Ld, doc_lengths, dev)
    codes = torch.empty(T, d, dtype=torch.uint8, device=dev)
    scales = torch.empty(T, dtype=torch.float16, device=dev)
    mins = torch.empty(T, dtype=torch.float16, device=dev)
    if T:
        lib = _lib.load()
        with _device_guard(dev):
            rc = lib.fmx_quantize_int8(
                _SRC_CODES[src.dtype], src.data_ptr(), src.stride(0), src.stride(1), B, Ld, d, lengths.data_ptr(),
                tok_group.data_ptr(), T, codes.data_ptr(), d, scales.data_ptr(), mins.data_ptr(), 0,
                _lib.stream_of(src),
            )
        _lib.check(rc)
    return PackedInt8Docs(codes, scales, mins, tok_group, lengths, max_len)


def flash_maxsim_packed(Q: torch.Tensor, docs: PackedDocs) -> torch.Tensor:
    """flash_maxsim over packed docs: float32 [B], equal to
    flash_maxsim(Q, D, lengths) on the padded docs."""
    assert Q.dim() == 2 and docs.tokens.dim() == 2 and Q.size(1) == docs.tokens.size(1)
    Lq, d = Q.shape
    B = docs.lengths.numel()
    kdt = _kernel_dtype(Q, docs.tokens)
    Qk, Dk = _prep(Q, kdt), _prep(docs.tokens, kdt)
    dev = _check_devices(Qk, Dk, docs.tok_group, docs.lengths)
    scores = torch.empty(B, device=dev, dtype=torch.float32)
    if B == 0:
        return scores
    if Lq == 0:
        return scores.zero_()
    if Dk.shape[0] == 0:  # every doc is empty
        return scores.fill_(float("-inf"))
    lib = _lib.load()
    Ld = max(docs.max_len, 1)
    nbytes = lib.fmx_fwd_packed_workspace_bytes(B, Lq, Ld, d)
    ws = _lib.workspace(nbytes, dev)
    with _device_guard(dev):
        rc = lib.fmx_fwd_packed(
            _lib.dtype_code(Qk), Qk.data_ptr(), Qk.stride(0), Lq, Dk.data_ptr(), Dk.stride(0), Dk.shape[0],
            docs.tok_group.data_ptr(), docs.lengths.data_ptr(), scores.data_ptr(), B, Ld, d, _lib.ptr(ws), nbytes,
            _lib.stream_of(Qk),
        )
    _lib.check(rc)
    return scores


def flash_maxsim_int8_packed(Q: torch.Tensor, docs: PackedInt8Docs) -> torch.Tensor:
    """flash_maxsim_int8 over packed uint8 docs: float32 [B], equal to
    flash_maxsim_int8(Q, codes, scales, mins, lengths) on the padded docs."""
    assert Q.dim() == 2 and docs.codes.dim() == 2 and Q.size(1) == docs.codes.size(1)
    Lq, d = Q.shape
    B = docs.lengths.numel()
    if docs.codes.dtype != torch.uint8:
        raise TypeError(f"codes must be torch.uint8, got {docs.codes.dtype}")
    Qk = _prep(Q, torch.float16)
    codes = _prep(docs.codes, None)
    scales = docs.scales.contiguous().half()
    mins = docs.mins.contiguous().half()
    dev = _check_devices(Qk, codes, scales, mins, docs.tok_group, docs.lengths)
    scores = torch.empty(B, device=dev, dtype=torch.float32)
    if B == 0:
        return scores
    if Lq == 0:
        return scores.zero_()
    if codes.shape[0] == 0:  # every doc is empty
        return scores.fill_(float("-inf"))
    lib = _lib.load()
    Ld = max(docs.max_len, 1)
    nbytes = lib.fmx_fwd_int8_packed_workspace_bytes(B, Lq, Ld, d)
    ws = _lib.workspace(nbytes, dev)
    with _device_guard(dev):
        rc = lib.fmx_fwd_int8_packed(
            Qk.data_ptr(), Qk.stride(0), Lq, codes.data_ptr(), codes.stride(0), scales.data_ptr(), mins.data_ptr(),
            codes.shape[0], docs.tok_group.data_ptr(), docs.lengths.data_ptr(), scores.data_ptr(), B, Ld, d,
            _lib.ptr(ws), nbytes, _lib.stream_of(Qk),
        )
    _lib.check(rc)
    return scores
