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

Docs may also be laid out longest first (sort_by_length=True): entry s of
tok_group and lengths then describes the s-th doc in memory (its slot) and
doc_ids[s] is that doc's number, to which the kernels write its score. Scores
are the same; variable-length docs scan faster that way, since workgroups
that run at once stream docs of similar length side by side.

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
    tok_group: torch.Tensor  # [B] int64: slot s starts at row 4 * tok_group[s]
    lengths: torch.Tensor    # [B] int32 valid tokens of slot s
    max_len: int             # max(lengths), the Ld of the padded equivalent
    doc_ids: torch.Tensor | None = None  # [B] int32: the doc in slot s (None: slot s is doc s)


class PackedInt8Docs(NamedTuple):
    """uint8 docs packed by quantize_int8_packed."""

    codes: torch.Tensor      # [T, d] uint8
    scales: torch.Tensor     # [T] fp16 per-token step
    mins: torch.Tensor       # [T] fp16 per-token minimum
    tok_group: torch.Tensor  # [B] int64, per slot as in PackedDocs
    lengths: torch.Tensor    # [B] int32, per slot
    max_len: int
    doc_ids: torch.Tensor | None = None  # [B] int32: the doc in slot s (None: slot s is doc s)


def _layout(B: int, Ld: int, doc_lengths, device, sort_by_length: bool = False):
    """(lengths int32 clamped to [0, Ld] and tok_group int64, both per doc;
    total rows T; max_len; the slot order: doc ids longest first (int64,
    stable among equal lengths) when sort_by_length, else None)."""
    if doc_lengths is None:
        lengths = torch.full((B,), Ld, dtype=torch.int32, device=device)
    else:
        assert doc_lengths.numel() == B, f"doc_lengths has {doc_lengths.numel()} entries, expected {B}"
        lengths = doc_lengths.to(device=device, dtype=torch.int32).reshape(B).clamp(0, Ld).contiguous()
    order = torch.sort(lengths, descending=True, stable=True).indices if sort_by_length and B > 0 else None
    groups = (lengths.to(torch.int64) + 3) // 4
    slot_groups = groups if order is None else groups[order]
    ends = torch.cumsum(slot_groups, 0)
    slot_start = ends - slot_groups
    if order is None:
        tok_group = slot_start.contiguous()
    else:
        tok_group = torch.empty_like(slot_start)
        tok_group[order] = slot_start
    T = 4 * int(ends[-1]) if B > 0 else 0
    max_len = int(lengths.max()) if B > 0 else 0
    return lengths, tok_group, T, max_len, order


def _slots(lengths, tok_group, order):
    """Per-slot lengths and tok_group, and doc_ids, from the per-doc ones."""
    if order is None:
        return lengths, tok_group, None
    return lengths[order].contiguous(), tok_group[order].contiguous(), order.to(torch.int32).contiguous()


def _ids(docs) -> tuple:
    """(doc_ids,) when the docs carry a slot order, checked as int32 [B]; else ()."""
    if docs.doc_ids is None:
        return ()
    ids = docs.doc_ids
    assert ids.dtype == torch.int32 and ids.numel() == docs.lengths.numel() and ids.is_contiguous(), (
        "doc_ids must be a contiguous int32 tensor with one entry per doc")
    return (ids,)


def pack_docs(D: torch.Tensor, doc_lengths=None, sort_by_length: bool = False) -> PackedDocs:
    """Packs the first doc_lengths[b] tokens of each doc of D [B, Ld, d]
    (all Ld when doc_lengths is None; lengths are clamped to [0, Ld]).
    Rows between a doc's length and its next 4-token boundary are zero.
    sort_by_length: lay the docs out longest first (doc_ids set)."""
    assert D.dim() == 3
    B, Ld, d = D.shape
    lengths, tok_group, T, max_len, order = _layout(B, Ld, doc_lengths, D.device, sort_by_length)
    tokens = torch.zeros(T, d, dtype=D.dtype, device=D.device)
    if T:
        j = torch.arange(Ld, device=D.device)
        valid = j[None, :] < lengths[:, None].to(torch.int64)
        rows = (4 * tok_group[:, None] + j[None, :])[valid]
        tokens[rows] = D[valid]
    slot_lengths, slot_group, doc_ids = _slots(lengths, tok_group, order)
    return PackedDocs(tokens, slot_group, slot_lengths, max_len, doc_ids)


def quantize_int8_packed(D: torch.Tensor, doc_lengths=None, sort_by_length: bool = False) -> PackedInt8Docs:
    """quantize_int8 of the first doc_lengths[b] tokens of each doc of D
    [B, Ld, d] (on the GPU), written straight into the packed layout by one
    pass of the HIP encoder: per token the codes, scale and min are bit-equal
    to quantize_int8(D)'s. sort_by_length: lay the docs out longest first
    (doc_ids set)."""
    assert D.dim() == 3
    B, Ld, d = D.shape
    src = _quant_source(D)
    dev = _check_devices(src)
    lengths, tok_group, T, max_len, order = _layout(B, Ld, doc_lengths, dev, sort_by_length)
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
    slot_lengths, slot_group, doc_ids = _slots(lengths, tok_group, order)
    return PackedInt8Docs(codes, scales, mins, slot_group, slot_lengths, max_len, doc_ids)


def flash_maxsim_packed(Q: torch.Tensor, docs: PackedDocs) -> torch.Tensor:
    """flash_maxsim over packed docs: float32 [B], equal to
    flash_maxsim(Q, D, lengths) on the padded docs."""
    assert Q.dim() == 2 and docs.tokens.dim() == 2 and Q.size(1) == docs.tokens.size(1)
    Lq, d = Q.shape
    B = docs.lengths.numel()
    kdt = _kernel_dtype(Q, docs.tokens)
    Qk, Dk = _prep(Q, kdt), _prep(docs.tokens, kdt)
    dev = _check_devices(Qk, Dk, docs.tok_group, docs.lengths, *_ids(docs))
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
            docs.tok_group.data_ptr(), docs.lengths.data_ptr(), _lib.ptr(docs.doc_ids), scores.data_ptr(), B, Ld, d,
            _lib.ptr(ws), nbytes, _lib.stream_of(Qk),
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
    dev = _check_devices(Qk, codes, scales, mins, docs.tok_group, docs.lengths, *_ids(docs))
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
            codes.shape[0], docs.tok_group.data_ptr(), docs.lengths.data_ptr(), _lib.ptr(docs.doc_ids),
            scores.data_ptr(), B, Ld, d,
            _lib.ptr(ws), nbytes, _lib.stream_of(Qk),
        )
    _lib.check(rc)
    return scores
