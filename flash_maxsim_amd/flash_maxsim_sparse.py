"""Sparse MaxSim: each doc scored with its own subset of query tokens.

Mirrors the reference module flash_maxsim/flash_maxsim_sparse.py:
flash_maxsim_sparse (:98-140) and maxsim_sparse_naive (:143-157). Doc b uses
query rows Q[indices[b, k]] for k < K; the HIP kernel gathers those rows into
its VGPR query tile directly from Q (no per-doc copy of Q is materialised).
"""

from __future__ import annotations

import torch

from . import _lib
from .flash_maxsim import _check_devices, _device_guard, _kernel_dtype, _lengths, _prep


def flash_maxsim_sparse(
    Q: torch.Tensor,
    D: torch.Tensor,
    indices: torch.Tensor,
    doc_lengths=None,
) -> torch.Tensor:
    """flash_maxsim where doc b only sees K chosen query tokens: float32 [B].

    Q is [Lq, d], D [B, Ld, d], indices [B, K] integer rows of Q for each doc
    (a row outside [0, Lq) contributes a zero query token), doc_lengths
    optional [B]. Reference signature: flash_maxsim_sparse.py:98.
    """
    assert Q.dim() == 2 and D.dim() == 3 and indices.dim() == 2
    Lq, d = Q.shape
    B, Ld, _ = D.shape
    _, K = indices.shape
    assert indices.shape[0] == B
    assert D.shape[2] == d

    dt = _kernel_dtype(Q, D)
    Q = _prep(Q, dt)
    D = _prep(D, dt)
    indices = indices.to(device=D.device, dtype=torch.int32).contiguous()
    lengths = _lengths(B, D.device, doc_lengths)
    dev = _check_devices(Q, D, indices, lengths)
    scores = torch.empty(B, device=dev, dtype=torch.float32)
    if B == 0:
        return scores
    if K == 0 or Lq == 0:
        return scores.zero_()

    lib = _lib.load()
    nbytes = lib.fmx_fwd_sparse_workspace_bytes(B, K, Ld, d)
    ws = _lib.workspace(nbytes, dev)
    with _device_guard(dev):
        rc = lib.fmx_fwd_sparse(
            _lib.dtype_code(Q), Q.data_ptr(), Q.stride(0), Lq, D.data_ptr(), D.stride(0), D.stride(1),
            indices.data_ptr(), indices.stride(0), indices.stride(1), K, _lib.ptr(lengths),
            scores.data_ptr(), B, Ld, d, _lib.ptr(ws), nbytes, _lib.stream_of(Q),
        )
    _lib.check(rc)
    return scores


def maxsim_sparse_naive(
    Q: torch.Tensor,
    D: torch.Tensor,
    indices: torch.Tensor,
) -> torch.Tensor:
    """Unfused float32 counterpart of flash_maxsim_sparse, for checking: [B]
    (reference flash_maxsim_sparse.py:143-157; indices must be valid rows)."""
    Q_sel = Q[indices.long()].float()  # [B, K, d]
    S = torch.matmul(Q_sel, D.float().transpose(1, 2).contiguous())  # [B, K, Ld]
    return S.max(dim=2).values.sum(dim=1)
