"""Writes the golden fixtures in tests/golden/ (run: python tests/golden/make_golden.py).

The reference ships no golden vectors, known-answer tests or fixtures for this
path (its tests compare to maxsim_naive at atol=1.0 on unseeded data). These
fixtures are built here:

  basis.npz      one-hot queries against scaled one-hot doc tokens with ragged
                 lengths (0, clamped, full): every score and argmax follows from
                 index arithmetic, written out by hand below.
  ties.npz       repeated doc tokens: exact ties, the first index must win.
  nan.npz        NaN doc and query tokens (torch.max's rule: NaN is the max,
                 the first NaN its index) and a NaN masked past a doc's length.
  quant.npz      rows on exact binary grids, a constant row (scale floor 1e-8,
                 which rounds to fp16 zero) and exact half-way codes (round half
                 to even): codes, fp16 scale and min follow by hand.
  bwd.npz        a 2-doc backward with a shared argmax row: dQ and dD by hand.
  random_small.npz  fp16-valued random inputs (batched, varlen, int8) with
                 expected values from the float64 NumPy restatement
                 (oracle/oracle_np.py): a regression pin for both oracles.

Values are in float32 holding fp16-exact numbers, so the same inputs feed the
fp16 GPU kernels unchanged.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))


def basis_case():
    B, Lq, Ld, d = 4, 8, 12, 16
    Q = np.zeros((Lq, d), np.float32)
    for q in range(Lq):
        Q[q, q] = 1.0
    D = np.zeros((B, Ld, d), np.float32)
    val = np.zeros((B, Ld), np.float64)
    hot = np.zeros((B, Ld), np.int64)
    for b in range(B):
        for j in range(Ld):
            sign = -1.0 if (j + b) % 3 == 0 else 1.0
            val[b, j] = sign * (j + 1) / 16.0
            hot[b, j] = (j + b) % d
            D[b, j, hot[b, j]] = val[b, j]
    lengths = np.array([12, 5, 0, 20], np.int32)  # full, ragged, empty, clamped to Ld
    scores = np.zeros(B)
    argmax = np.zeros((B, Lq), np.int32)
    for b in range(B):
        n = min(max(int(lengths[b]), 0), Ld)
        if n == 0:
            scores[b] = -np.inf
            continue
        for q in range(Lq):
            # S[q, j] = val[b, j] if token j is hot on dim q, else 0.
            s = [val[b, j] if hot[b, j] == q else 0.0 for j in range(n)]
            m = max(s)
            scores[b] += m
            argmax[b, q] = s.index(m)
    return dict(Q=Q, D=D, lengths=lengths, scores=scores, argmax=argmax)


def ties_case():
    B, Lq, Ld, d = 2, 4, 10, 8
    Q = np.zeros((Lq, d), np.float32)
    for q in range(Lq):
        Q[q, q] = 1.0
    D = np.zeros((B, Ld, d), np.float32)
    for b in range(B):
        for j in range(Ld):
            D[b, j, j % 4] = 1.0  # token j repeats every 4 positions
    lengths = np.array([10, 2], np.int32)
    # Doc 0: S[q, j] = 1 at j = q, q+4, q+8 -> first index q, score 4.
    # Doc 1 (len 2): q=0 -> j=0, q=1 -> j=1, q=2,3 -> all zero, first index 0; score 2.
    scores = np.array([4.0, 2.0])
    argmax = np.array([[0, 1, 2, 3], [0, 1, 0, 0]], np.int32)
    return dict(Q=Q, D=D, lengths=lengths, scores=scores, argmax=argmax)


def nan_case():
    """NaN handling of maxsim_naive's torch.max (flash_maxsim.py:301): a NaN
    similarity is the max of its row and the first NaN's index is the argmax;
    a NaN past a doc's length is masked to -inf first (:297-300)."""
    B, Lq, Ld, d = 4, 4, 8, 8
    nan = np.float32(np.nan)
    Q = np.zeros((Lq, d), np.float32)
    for q in range(Lq):
        Q[q, q] = 1.0
    D = np.zeros((B, Ld, d), np.float32)
    for b in range(B):
        for j in range(Ld):
            D[b, j, j % 4] = (j + 1) / 8.0  # S[q, j] = (j + 1) / 8 when j % 4 == q, else 0
    D[0, 5, 7] = nan                  # doc 0: token 5 is NaN against every query token
    D[1, 6, 0] = nan                  # doc 1 (length 4): the NaN token is masked
    D[2, 6, 3] = nan                  # doc 2: NaN tokens 3 and 6, the first is 3
    D[2, 3, 5] = nan
    D[3, 0, 0] = nan                  # doc 3: empty, its NaN never read
    lengths = np.array([8, 4, 8, 0], np.int32)
    # doc 1: S[q, q] = (q + 1) / 8 is its only nonzero: 1/8 + 2/8 + 3/8 + 4/8.
    scores = np.array([np.nan, 1.25, np.nan, -np.inf])
    argmax = np.array([[5] * 4, [0, 1, 2, 3], [3] * 4, [0] * 4], np.int32)
    # A query token with a NaN (token 2) is NaN against every doc token: its
    # argmax is the doc's first token and every non-empty doc scores NaN.
    Qnan = Q.copy()
    Qnan[2, 6] = nan
    scores_qnan = np.array([np.nan, np.nan, np.nan, -np.inf])
    argmax_qnan = argmax.copy()
    argmax_qnan[:, 2] = 0
    return dict(Q=Q, D=D, lengths=lengths, scores=scores, argmax=argmax, Qnan=Qnan, scores_qnan=scores_qnan,
                argmax_qnan=argmax_qnan)


def quant_case():
    d = 256
    k = np.arange(d, dtype=np.float64)
    rows = np.zeros((5, d), np.float32)
    codes = np.zeros((5, d), np.uint8)
    scale16 = np.zeros(5, np.float16)
    min16 = np.zeros(5, np.float16)
    # Row 0: -1 + k/128: min -1, max 255/128 - 1, scale exactly 2^-7, codes k.
    rows[0] = -1.0 + k / 128.0
    codes[0] = np.arange(d)
    scale16[0], min16[0] = 2.0**-7, -1.0
    # Row 1: constant 0.5: scale clamps to 1e-8 (fp16 rounds it to 0), codes 0.
    rows[1] = 0.5
    scale16[1], min16[1] = 0.0, 0.5
    # Row 2: min 0, max 255/16 -> scale 1/16; 2.5 and 3.5 steps round half to even.
    rows[2] = 0.0
    rows[2, 1] = 255.0 / 16.0
    rows[2, 2] = 2.5 / 16.0
    rows[2, 3] = 3.5 / 16.0
    rows[2, 4] = 0.5 / 16.0
    codes[2, 1], codes[2, 2], codes[2, 3], codes[2, 4] = 255, 2, 4, 0
    scale16[2], min16[2] = 1.0 / 16.0, 0.0
    # Row 3: -3 + k/64: scale 2^-6, codes k.
    rows[3] = -3.0 + k / 64.0
    codes[3] = np.arange(d)
    scale16[3], min16[3] = 2.0**-6, -3.0
    # Row 4: two values 1 and 3 only: scale 2/255 (not a binary fraction),
    # codes 0 and 255 exactly; fp16 scale is the rounding of float32(2/255).
    rows[4] = 1.0
    rows[4, ::2] = 3.0
    codes[4] = 0
    codes[4, ::2] = 255
    scale16[4], min16[4] = np.float16(np.float32(2.0) / np.float32(255.0)), 1.0
    return dict(D=rows.reshape(1, 5, d), codes=codes.reshape(1, 5, d),
                scales=scale16.reshape(1, 5, 1), mins=min16.reshape(1, 5, 1))


def bwd_case():
    Q = np.array([[1.0, 2.0, 0.5], [-1.0, 0.25, 3.0]], np.float32)  # [Lq=2, d=3]
    D = np.arange(2 * 3 * 3, dtype=np.float32).reshape(2, 3, 3) / 8.0  # [B=2, Ld=3, d=3]
    argmax = np.array([[1, 1], [0, 2]], np.int32)
    g = np.array([2.0, -1.0])
    dQ = np.zeros((2, 3))
    dD = np.zeros((2, 3, 3))
    for q in range(2):
        dQ[q] = 2.0 * D[0, 1] + (-1.0) * D[1, argmax[1, q]]
    dD[0, 1] = 2.0 * (Q[0] + Q[1])  # both tokens of doc 0 picked row 1
    dD[1, 0] = -1.0 * Q[0]
    dD[1, 2] = -1.0 * Q[1]
    return dict(Q=Q, D=D, argmax=argmax, grad=g, dQ=dQ, dD=dD)


def random_small_case():
    from oracle.oracle_np import dequantize_np, maxsim_np, quantize_np

    rng = np.random.default_rng(20261201)
    Nq, Lq, B, Ld, d = 2, 5, 3, 7, 24

    def norm16(shape):
        x = rng.standard_normal(shape).astype(np.float32)
        x /= np.linalg.norm(x, axis=-1, keepdims=True)
        return x.astype(np.float16).astype(np.float32)

    Q = norm16((Nq, Lq, d))
    D = norm16((B, Ld, d))
    lengths = np.array([7, 3, 1], np.int32)
    scores, argmax, _ = maxsim_np(Q, D, lengths)
    codes, s16, m16, _ = quantize_np(D)
    Dq = dequantize_np(codes, s16, m16)
    scores_int8, _, _ = maxsim_np(Q[0], Dq, lengths)
    return dict(Q=Q, D=D, lengths=lengths, scores=scores, argmax=argmax, codes=codes, scales=s16,
                mins=m16, scores_int8=scores_int8[0])


CASES = {"basis": basis_case, "ties": ties_case, "nan": nan_case, "quant": quant_case, "bwd": bwd_case,
         "random_small": random_small_case}


def main(names=None):
    for name in names or CASES:
        np.savez(HERE / f"{name}.npz", **CASES[name]())
        print("wrote", HERE / f"{name}.npz")


if __name__ == "__main__":
    main(sys.argv[1:])
