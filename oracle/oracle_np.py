"""Independent NumPy restatement of the oracle (vectorised, float64).

TEST INFRASTRUCTURE ONLY. It shares no code with maxsim_oracle.c; the two are
checked against each other and against closed-form cases in
tests/test_oracle.py, so that a slip in either shows up.

  maxsim_np      flash_maxsim/flash_maxsim.py:294-301 (+ argmax :132-135,
                 batched :233-250, sparse flash_maxsim_sparse.py:153-157)
  quantize_np    flash_maxsim/flash_maxsim_quant.py:23-28 (float32 arithmetic)
  dequantize_np  flash_maxsim/flash_maxsim_quant.py:31-33
  dequantize_fp16_np
                 flash_maxsim/flash_maxsim_quant.py:89 (the kernel's fp16
                 dequantisation before its dot product)
  bwd_np         flash_maxsim/flash_maxsim.py:153-188
"""

from __future__ import annotations

import numpy as np


def maxsim_np(Q, D, lengths=None, *, shared_docs=True, qidx=None):
    """(scores [Nq, B], argmax [Nq*B, Lq], best [Nq*B, Lq]) in float64."""
    Q = np.asarray(Q, dtype=np.float64)
    if Q.ndim == 2:
        Q = Q[None]
    D = np.asarray(D, dtype=np.float64)
    Nq, Lq_rows, d = Q.shape
    Bp, Ld, _ = D.shape
    B = Bp if shared_docs else Bp // Nq
    lens = np.full(Bp, Ld, dtype=np.int64) if lengths is None else np.clip(np.asarray(lengths, np.int64), 0, Ld)
    if qidx is not None:
        qidx = np.asarray(qidx, dtype=np.int64)
        Lq = qidx.shape[1]
    else:
        Lq = Lq_rows
    scores = np.empty((Nq, B))
    argmax = np.zeros((Nq * B, Lq), dtype=np.int32)
    best = np.empty((Nq * B, Lq))
    pos = np.arange(Ld)
    for qi in range(Nq):
        for b in range(B):
            drow = b if shared_docs else qi * B + b
            if qidx is not None:
                idx = qidx[b]
                valid = (idx >= 0) & (idx < Lq_rows)
                qm = np.where(valid[:, None], Q[qi][np.clip(idx, 0, Lq_rows - 1)], 0.0)
            else:
                qm = Q[qi]
            S = qm @ D[drow].T  # [Lq, Ld]
            S = np.where(pos[None, :] < lens[drow], S, -np.inf)
            item = qi * B + b
            if Ld > 0 and lens[drow] > 0:
                argmax[item] = np.argmax(S, axis=1)  # first occurrence of the max
                best[item] = S.max(axis=1)
            else:
                best[item] = -np.inf
            scores[qi, b] = best[item].sum()
    return scores, argmax, best


def quantize_np(D):
    """(codes uint8, scale fp16 [..., 1], min fp16 [..., 1], scale fp32 [..., 1])."""
    Df = np.asarray(D, dtype=np.float32)
    mn = Df.min(axis=-1, keepdims=True)
    mx = Df.max(axis=-1, keepdims=True)
    s = np.maximum((mx - mn) / np.float32(255.0), np.float32(1e-8))
    codes = np.clip(np.rint((Df - mn) / s), 0, 255).astype(np.uint8)
    return codes, s.astype(np.float16), mn.astype(np.float16), s


def dequantize_np(codes, scales, mins):
    """codes * scale + min in float32, as torch's dequantize_int8."""
    return (np.asarray(codes).astype(np.float32) * np.asarray(scales, dtype=np.float32)
            + np.asarray(mins, dtype=np.float32))


def dequantize_fp16_np(codes, scales, mins):
    """codes * scale + min rounded once to fp16 (float16 array).

    The product and sum are exact in float64 (an 8-bit code times an 11-bit
    significand, plus an fp16 min, spans fewer than 53 bits), so the cast is
    the single round-to-nearest-even of the exact value."""
    exact = (np.asarray(codes).astype(np.float64) * np.asarray(scales, dtype=np.float16).astype(np.float64)
             + np.asarray(mins, dtype=np.float16).astype(np.float64))
    with np.errstate(over="ignore"):  # past the fp16 range: inf, as the hardware rounds
        return exact.astype(np.float16)


def bwd_np(Q, D, argmax, grad):
    """(dQ [Lq, d], dD [B, Ld, d]) in float64."""
    Q = np.asarray(Q, dtype=np.float64)
    D = np.asarray(D, dtype=np.float64)
    B, Ld, d = D.shape
    Lq = Q.shape[0]
    am = np.asarray(argmax, dtype=np.int64).reshape(B, Lq)
    g = np.asarray(grad, dtype=np.float64)
    dQ = np.einsum("b,bqk->qk", g, D[np.arange(B)[:, None], am])
    dD = np.zeros((B, Ld, d))
    for b in range(B):
        np.add.at(dD[b], am[b], g[b] * Q)
    return dQ, dD
