"""MaxSim scoring on MI355X: single-query, batched and training entry points.

Mirrors the public functions of the reference module
flash_maxsim/flash_maxsim.py (flash_maxsim :221, flash_maxsim_batched :233,
flash_maxsim_train :289, maxsim_naive :294): same names, positional order,
defaults, AssertionError on bad ranks/shapes and fp16 casting of inputs. The
work runs in libflashmaxsim's HIP kernels (include/fmx.h); there is no CPU or
torch fallback for the flash_* functions.

Differences by design:
  * bfloat16 Q and D run on the bf16 MFMA as they are instead of being cast to
    fp16 (any other dtype mix is cast to fp16 as in the reference);
  * doc_lengths are clamped to [0, Ld] on the GPU (the reference reads past the
    doc for lengths > Ld) and must have one entry per doc row;
  * operands are read in place when their row strides are multiple of 8
    elements (d masked in the kernels), so D = store[..., :d] of a store padded
    to a multiple of 8 costs no copy; other layouts, and contiguous rows with
    d % 8 != 0, are copied once per call with d zero-padded to a multiple of 8
    (the kernels read rows with 16-byte loads).
"""

from __future__ import annotations

import contextlib

import torch
import torch.nn.functional as F

from . import _lib


def _check_devices(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(f"flash_maxsim_amd runs on a ROCm GPU; got a tensor on {dev}")
    for t in tensors[1:]:
        if t is not None and t.device != dev:
            raise RuntimeError(f"all operands must be on {dev}; got one on {t.device}")
    return dev


def _device_guard(dev: torch.device):
    if dev.index is None or dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


def _kernel_dtype(*tensors: torch.Tensor) -> torch.dtype:
    """fp16, as the reference's .half() casts, unless every operand is bf16."""
    return torch.bfloat16 if all(t.dtype == torch.bfloat16 for t in tensors) else torch.float16


def _abi_ready(t: torch.Tensor, dtype: torch.dtype | None) -> bool:
    """True when the kernels can read t in place: kernel dtype, unit stride
    along d, every other stride a multiple of 8 elements and at least d along
    rows, 16-byte aligned. The kernels mask elements at or past d, so rows of a
    wider buffer (t = buf[..., :d]) need no copy even when d % 8 != 0."""
    if t.dim() < 2 or (dtype is not None and t.dtype != dtype):
        return False
    if t.stride(-1) != 1 or t.stride(-2) < t.shape[-1] or t.data_ptr() % 16:
        return False
    return all(s % 8 == 0 for s in t.stride()[:-1])


def _prep(t: torch.Tensor, dtype: torch.dtype | None) -> torch.Tensor:
    """t itself when the kernels can read it in place, else a contiguous cast
    copy with d zero-padded to a multiple of 8, 16-byte aligned."""
    if _abi_ready(t, dtype):
        return t
    t = t.contiguous()
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    pad = (-t.shape[-1]) % 8
    if pad:
        t = F.pad(t, (0, pad))
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _lengths(total: int, device: torch.device, doc_lengths) -> torch.Tensor | None:
    """int32 doc lengths on the device, or None for full length (reference :211-214)."""
    if doc_lengths is None:
        return None
    lengths = doc_lengths.to(device=device, dtype=torch.int32).contiguous()
    assert lengths.numel() == total, f"doc_lengths has {lengths.numel()} entries, expected {total}"
    return lengths


def _launch_fwd(Q, D, lengths, Nq, B, Lq, Ld, d, shared_docs, save_argmax):
    """Scores [Nq, B] fp32 (+ argmax [Nq*B, Lq] int32) from prepared operands.

    Q is [Nq, Lq, d'] or [Lq, d'], D is [B', Ld, d'] with d' >= d (the
    kernels read the first d elements of each row; strides as _prep leaves
    them); mirrors _launch_fwd (reference flash_maxsim.py:195-208).
    """
    dev = _check_devices(Q, D, lengths)
    lib = _lib.load()
    scores = torch.empty(Nq, B, device=dev, dtype=torch.float32)
    argmax = torch.empty(Nq * B, Lq, device=dev, dtype=torch.int32) if save_argmax else None
    if Nq == 0 or B == 0:
        return scores, argmax
    if Lq == 0:
        scores.zero_()
        return scores, argmax
    nbytes = lib.fmx_fwd_workspace_bytes(Nq, B, Lq, Ld, d)
    ws = _lib.workspace(nbytes, dev)
    q_stride_n = Q.stride(0) if Q.dim() == 3 else 0
    with _device_guard(dev):
        rc = lib.fmx_fwd(
            _lib.dtype_code(Q), Q.data_ptr(), q_stride_n, Q.stride(-2),
            D.data_ptr(), D.stride(0), D.stride(1), _lib.ptr(lengths),
            scores.data_ptr(), scores.stride(0), scores.stride(1), _lib.ptr(argmax),
            Nq, B, Lq, Ld, d, int(bool(shared_docs)), _lib.ptr(ws), nbytes, _lib.stream_of(Q),
        )
    _lib.check(rc)
    return scores, argmax


def flash_maxsim(Q: torch.Tensor, D: torch.Tensor, doc_lengths=None) -> torch.Tensor:
    """Scores one query against every doc: float32 [B].

    Q is [Lq, d], D is [B, Ld, d]; score[b] adds up, over the query tokens, the
    best similarity among doc b's first doc_lengths[b] tokens (all Ld when
    doc_lengths is None). Reference signature: flash_maxsim.py:221.
    """
    assert Q.ndim == 2 and D.ndim == 3 and Q.size(1) == D.size(2)
    Lq, d = Q.shape
    B, Ld = D.shape[:2]
    kdt = _kernel_dtype(Q, D)
    lengths = _lengths(B, D.device, doc_lengths)
    scores, _ = _launch_fwd(_prep(Q, kdt).unsqueeze(0), _prep(D, kdt), lengths, 1, B, Lq, Ld, d, True, False)
    return scores[0]


def flash_maxsim_batched(Q: torch.Tensor, D: torch.Tensor, doc_lengths=None,
                         shared_docs: bool = True) -> torch.Tensor:
    """Scores Nq queries at once: float32 [Nq, B].

    Q is [Nq, Lq, d]. With shared_docs every query meets the same docs D
    [B, Ld, d]; otherwise query i has its own docs D[i] of D [Nq, B, Ld, d] and
    doc_lengths, if given, holds Nq*B entries in that order. Reference
    signature: flash_maxsim.py:233.
    """
    assert Q.ndim == 3 and Q.size(2) == D.size(-1)
    Nq, Lq, d = Q.shape
    if shared_docs:
        assert D.ndim == 3
        B, Ld = D.shape[:2]
        doc_rows = D
    else:
        assert D.ndim == 4 and D.size(0) == Nq
        B, Ld = D.shape[1:3]
        doc_rows = D.reshape(Nq * B, Ld, d)
    kdt = _kernel_dtype(Q, doc_rows)
    lengths = _lengths(doc_rows.size(0), D.device, doc_lengths)
    scores, _ = _launch_fwd(_prep(Q, kdt), _prep(doc_rows, kdt), lengths, Nq, B, Lq, Ld, d, shared_docs, False)
    return scores


class _FlashMaxSimFn(torch.autograd.Function):
    """Autograd node of flash_maxsim_train / flash_maxsim_train_batched
    (reference flash_maxsim.py:253-286, extended to Nq queries and doc lengths).

    The forward kernel records, for every (query, doc, query token), the first
    doc token reaching the max; the gradient of a max flows only to that token,
    so the backward is a gather (dQ) and a scatter (dD) through those indices.
    Docs of length 0 score -inf and get and give no gradient, as in autograd
    through maxsim_naive.
    """

    @staticmethod
    def forward(ctx, Q, D, lengths):
        batched = Q.ndim == 3
        Q3 = Q if batched else Q.unsqueeze(0)
        Nq, Lq, d = Q3.shape
        B, Ld = D.shape[:2]
        kdt = _kernel_dtype(Q, D)
        Qk, Dk = _prep(Q3, kdt), _prep(D, kdt)
        scores, argmax = _launch_fwd(Qk, Dk, lengths, Nq, B, Lq, Ld, d, True, True)
        ctx.save_for_backward(Qk, Dk, argmax, lengths)
        ctx.d = d
        ctx.batched = batched
        return scores if batched else scores[0]

    @staticmethod
    def backward(ctx, grad_scores):
        Qk, Dk, argmax, lengths = ctx.saved_tensors
        d = ctx.d
        Nq, Lq = Qk.shape[:2]
        B, Ld = Dk.shape[:2]
        need_q, need_d = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dev = _check_devices(Qk, Dk, grad_scores)
        grad_Q = torch.empty(Nq, Lq, d, device=dev, dtype=Qk.dtype) if need_q else None
        grad_D = torch.empty(B, Ld, d, device=dev, dtype=Dk.dtype) if need_d else None
        if (grad_Q is None and grad_D is None) or Lq == 0 or Ld == 0 or B == 0:
            if grad_Q is not None:
                grad_Q.zero_()
            if grad_D is not None:
                grad_D.zero_()
        else:
            # fp32 gradient read in place through its strides (the expanded
            # gradient of scores.sum() has stride 0: no copy).
            g = grad_scores.float().reshape(Nq, B) if not ctx.batched else grad_scores.float()
            if g.dim() == 1:
                g = g.unsqueeze(0)
            lib = _lib.load()
            nbytes = lib.fmx_bwd_batched_workspace_bytes(Nq, B, Lq, Ld, d)
            ws = _lib.workspace(nbytes, dev)
            with _device_guard(dev):
                rc = lib.fmx_bwd_batched(
                    _lib.dtype_code(Qk), Qk.data_ptr(), Qk.stride(0), Qk.stride(1), Dk.data_ptr(), Dk.stride(0),
                    Dk.stride(1), _lib.ptr(lengths), argmax.data_ptr(), g.data_ptr(), g.stride(0), g.stride(1),
                    _lib.ptr(grad_Q), _lib.ptr(grad_D), Nq, B, Lq, Ld, d, _lib.ptr(ws), nbytes, _lib.stream_of(Qk),
                )
            _lib.check(rc)
        if grad_Q is not None and not ctx.batched:
            grad_Q = grad_Q[0]
        return grad_Q, grad_D, None


def flash_maxsim_train(Q: torch.Tensor, D: torch.Tensor, doc_lengths=None) -> torch.Tensor:
    """flash_maxsim differentiable in Q and D: float32 [B].

    Gradients come back in the kernel dtype (fp16, or bf16 for bf16 inputs);
    autograd casts them to the leaves' dtypes. Reference signature:
    flash_maxsim.py:289 (Q, D); doc_lengths is an extension (the reference
    trains on full-length docs only, :260).
    """
    assert Q.ndim == 2 and D.ndim == 3 and Q.size(1) == D.size(2)
    return _FlashMaxSimFn.apply(Q, D, _lengths(D.size(0), D.device, doc_lengths))


def flash_maxsim_train_batched(Q: torch.Tensor, D: torch.Tensor, doc_lengths=None) -> torch.Tensor:
    """Nq queries against shared docs, differentiable in Q and D: float32
    [Nq, B] (the scores of flash_maxsim_batched with shared_docs=True).
    Extension: the reference trains one query at a time (flash_maxsim.py:289)."""
    assert Q.ndim == 3 and D.ndim == 3 and Q.size(2) == D.size(2)
    return _FlashMaxSimFn.apply(Q, D, _lengths(D.size(0), D.device, doc_lengths))


def maxsim_naive(Q: torch.Tensor, D: torch.Tensor, doc_lengths=None) -> torch.Tensor:
    """Unfused float32 MaxSim in plain torch, for checking: [B].

    Materialises every similarity, S = D Q^T per doc, masks doc tokens at or
    past doc_lengths to -inf, takes the max over doc tokens and sums over
    query tokens (reference flash_maxsim.py:294-301). Runs wherever its inputs
    live, CPU included.
    """
    S = torch.matmul(D.float(), Q.float().t().contiguous())  # [B, Ld, Lq]
    if doc_lengths is not None:
        Ld = D.shape[1]
        pos = torch.arange(Ld, device=D.device)[None, :, None]
        S = S.masked_fill(pos >= doc_lengths.to(D.device)[:, None, None], float("-inf"))
    return S.max(dim=1).values.sum(dim=1)
