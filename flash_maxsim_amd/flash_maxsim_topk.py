"""Top-k retrieval on the GPU: score, then select the k best docs per query.

Callers of the reference rank flash_maxsim's scores right after computing
them (torch topk / argsort over its output); these functions do the scoring
and that selection in libflashmaxsim's kernels, back to back on the current
stream. Extension of the reference API (no counterpart in flash_maxsim 0.1.0).

Ranking: score descending, NaN before every number (as torch.topk ranks NaN),
equal scores by the smaller doc index; k <= min(B, 8192). Values equal
torch.topk(scores, k).values; indices are torch.topk's up to the tie order,
which is fixed here (smaller index first).
"""

from __future__ import annotations

import torch

from . import _lib
from .flash_maxsim import (_check_devices, _device_guard, _kernel_dtype, _lengths, _prep, flash_maxsim,
                           flash_maxsim_batched)
from .flash_maxsim_quant import flash_maxsim_int8

def topk_scores(scores: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(values fp32, indices int64) of the k best entries of each row of
    scores ([B] or [Nq, B], on the GPU), best first."""
    assert scores.dim() in (1, 2)
    rows = scores.reshape(1, -1) if scores.dim() == 1 else scores
    Nq, B = rows.shape
    if not 0 <= k <= B:
        raise ValueError(f"k={k} must be in [0, {B}]")
    rows = rows.to(torch.float32)
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    dev = _check_devices(rows)
    values = torch.empty(Nq, k, device=dev, dtype=torch.float32)
    indices = torch.empty(Nq, k, device=dev, dtype=torch.int64)
    if Nq and k:
        lib = _lib.load()
        nbytes = lib.fmx_topk_workspace_bytes(Nq, B, k)
        ws = _lib.workspace(nbytes, dev)
        with _device_guard(dev):
            rc = lib.fmx_topk(rows.data_ptr(), rows.stride(0), Nq, B, k, values.data_ptr(), indices.data_ptr(), k,
                              _lib.ptr(ws), nbytes, _lib.stream_of(rows))
        _lib.check(rc)
    if scores.dim() == 1:
        return values[0], indices[0]
    return values, indices


def flash_maxsim_topk(Q: torch.Tensor, D: torch.Tensor, k: int, doc_lengths=None):
    """The k best docs for one query: (scores fp32 [k], doc indices int64 [k]).

    One call of fmx_fwd_topk (the scoring and the selection kernels back to
    back); the results equal topk_scores(flash_maxsim(Q, D), k).
    """
    assert Q.ndim == 2 and D.ndim == 3 and Q.size(1) == D.size(2)
    Lq, d = Q.shape
    B, Ld = D.shape[:2]
    if not 0 <= k <= B:
        raise ValueError(f"k={k} must be in [0, {B}]")
    if Lq == 0 or k == 0:
        return topk_scores(flash_maxsim(Q, D, doc_lengths), k)
    kdt = _kernel_dtype(Q, D)
    lengths = _lengths(B, D.device, doc_lengths)
    Qk, Dk = _prep(Q, kdt), _prep(D, kdt)
    dev = _check_devices(Qk, Dk, lengths)
    scores = torch.empty(B, device=dev, dtype=torch.float32)
    values = torch.empty(k, device=dev, dtype=torch.float32)
    indices = torch.empty(k, device=dev, dtype=torch.int64)
    lib = _lib.load()
    with _device_guard(dev):
        stream = _lib.stream_of(Qk)
        nbytes = lib.fmx_fwd_topk_workspace_bytes(B, Lq, Ld, d, k)
        ws = _lib.workspace(nbytes, dev)
        rc = lib.fmx_fwd_topk(_lib.dtype_code(Qk), Qk.data_ptr(), Qk.stride(0), Dk.data_ptr(), Dk.stride(0),
                              Dk.stride(1), _lib.ptr(lengths), B, Lq, Ld, d, k, scores.data_ptr(), values.data_ptr(),
                              indices.data_ptr(), _lib.ptr(ws), nbytes, stream)
    _lib.check(rc)
    return values, indices


def flash_maxsim_batched_topk(Q: torch.Tensor, D: torch.Tensor, k: int, doc_lengths=None,
                              shared_docs: bool = True):
    """The k best docs for each of Nq queries: ([Nq, k] fp32, [Nq, k] int64)."""
    return topk_scores(flash_maxsim_batched(Q, D, doc_lengths, shared_docs), k)


def flash_maxsim_int8_topk(Q: torch.Tensor, D_uint8: torch.Tensor, scales: torch.Tensor, mins: torch.Tensor,
                           k: int, doc_lengths=None):
    """The k best uint8-encoded docs for one query: ([k] fp32, [k] int64)."""
    return topk_scores(flash_maxsim_int8(Q, D_uint8, scales, mins, doc_lengths), k)
