"""CPU oracle for flash_maxsim's scoring path (ctypes over liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. The product package
flash_maxsim_amd never imports it.

The C restatement (maxsim_oracle.c) accumulates similarities in double and
reproduces quantize_int8's float32 arithmetic bit for bit; oracle_np.py is an
independent NumPy restatement used to pin it. Each function cites the
reference lines it follows in maxsim_oracle.c.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_lib = None


def build() -> Path:
    """Compiles liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "liboracle.so"], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run `make -C oracle`")
        lib = ctypes.CDLL(str(LIB_PATH))
        p, i64, i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.oracle_maxsim.restype = None
        lib.oracle_maxsim.argtypes = [p, p, p, p, i64, i64, i64, i64, i64, i64, i, p, p, p, i]
        lib.oracle_maxsim_int8.restype = None
        lib.oracle_maxsim_int8.argtypes = [p, p, p, p, p, i64, i64, i64, i64, p, i]
        lib.oracle_quantize_int8.restype = None
        lib.oracle_quantize_int8.argtypes = [p, i64, i64, p, p, p, p]
        lib.oracle_bwd.restype = None
        lib.oracle_bwd.argtypes = [p, p, p, p, i64, i64, i64, i64, p, p]
        lib.oracle_f32_to_f16.restype = ctypes.c_uint16
        lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        _lib = lib
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i32(a) -> np.ndarray | None:
    return None if a is None else np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def default_threads() -> int:
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        return max(1, os.cpu_count() or 1)


def maxsim(Q, D, lengths=None, *, shared_docs=True, qidx=None, want_argmax=False, nthreads=None):
    """Scores [Nq, B] (float64) of Q [Nq, Lq, d] (or [Lq, d]) against D.

    D is [B, Ld, d] (shared_docs) or [Nq*B, Ld, d]; lengths has one entry per
    doc row. qidx [B, K] scores doc b with query rows qidx[b] (sparse; Nq = 1).
    With want_argmax also returns argmax [Nq*B, Lq'] (int32, first max) and the
    max similarities [Nq*B, Lq'] (float64).
    """
    Q = _f32(Q)
    if Q.ndim == 2:
        Q = Q[None]
    D = _f32(D)
    Nq, Lq_rows, d = Q.shape
    Bp, Ld, d2 = D.shape
    assert d == d2
    B = Bp if shared_docs else Bp // Nq
    qidx = _i32(qidx)
    Lq = qidx.shape[1] if qidx is not None else Lq_rows
    lengths = _i32(lengths)
    scores = np.empty((Nq, B), dtype=np.float64)
    argmax = np.empty((Nq * B, Lq), dtype=np.int32) if want_argmax else None
    best = np.empty((Nq * B, Lq), dtype=np.float64) if want_argmax else None
    _load().oracle_maxsim(_p(Q), _p(D), _p(lengths), _p(qidx), Nq, B, Lq, Lq_rows, Ld, d,
                          int(bool(shared_docs)), _p(scores), _p(argmax), _p(best),
                          nthreads or default_threads())
    if want_argmax:
        return scores, argmax, best
    return scores


def maxsim_int8(Q, codes, scales, mins, lengths=None, nthreads=None):
    """Single-query scores [B] (float64) against dequantize_int8(codes, scales, mins)."""
    Q = _f32(Q)
    codes = np.ascontiguousarray(np.asarray(codes, dtype=np.uint8))
    B, Ld, d = codes.shape
    scales = _f32(np.asarray(scales).reshape(B, Ld))
    mins = _f32(np.asarray(mins).reshape(B, Ld))
    lengths = _i32(lengths)
    scores = np.empty(B, dtype=np.float64)
    _load().oracle_maxsim_int8(_p(Q), _p(codes), _p(scales), _p(mins), _p(lengths), B, Q.shape[0], Ld, d,
                               _p(scores), nthreads or default_threads())
    return scores


def quantize_int8(D):
    """(codes uint8 [..., d], scale fp16 [..., 1], min fp16 [..., 1], scale fp32 [..., 1])."""
    D = _f32(D)
    lead = D.shape[:-1]
    d = D.shape[-1]
    rows = int(np.prod(lead)) if lead else 1
    codes = np.empty(D.shape, dtype=np.uint8)
    sh = np.empty(lead + (1,), dtype=np.uint16)
    mh = np.empty(lead + (1,), dtype=np.uint16)
    sf = np.empty(lead + (1,), dtype=np.float32)
    _load().oracle_quantize_int8(_p(D), rows, d, _p(codes), _p(sh), _p(mh), _p(sf))
    return codes, sh.view(np.float16), mh.view(np.float16), sf


def f32_to_f16_bits(x: float) -> int:
    return int(_load().oracle_f32_to_f16(float(x)))


def bwd(Q, D, argmax, grad, want_dD=True):
    """(dQ [Lq, d], dD [B, Ld, d]) in float64 for the single-query argmax backward.

    With want_dD=False only dQ is formed (dD is None): the C function skips a
    NULL output, so dQ of docs too large to hold dD for costs no B*Ld*d array.
    """
    Q = _f32(Q)
    D = _f32(D)
    B, Ld, d = D.shape
    Lq = Q.shape[0]
    am = _i32(argmax).reshape(B, Lq)
    g = np.ascontiguousarray(np.asarray(grad, dtype=np.float64))
    dQ = np.empty((Lq, d), dtype=np.float64)
    dD = np.empty((B, Ld, d), dtype=np.float64) if want_dD else None
    _load().oracle_bwd(_p(Q), _p(D), _p(am), _p(g), B, Lq, Ld, d, _p(dQ), _p(dD))
    return dQ, dD


def topk(scores, k):
    """(values float32 [..., k], indices int64 [..., k]) of each row's k best
    scores: descending, NaN first (torch.topk ranks NaN above every number),
    equal scores by smaller index. Restates the ranking callers apply to
    flash_maxsim's output (torch topk / argsort, e.g. reference
    benchmarks/bench.py:36, examples/demo.py:127-128) with the tie order fixed.
    """
    s = np.asarray(scores, dtype=np.float32)
    rows = s.reshape(-1, s.shape[-1])
    B = rows.shape[1]
    idx = np.arange(B)
    vals, inds = [], []
    for r in rows:
        nan = np.isnan(r)
        neg = np.where(nan, 0.0, -r.astype(np.float64))
        order = np.lexsort((idx, neg, ~nan))[:k]  # NaN first, then value desc, then index
        vals.append(r[order])
        inds.append(order.astype(np.int64))
    shape = s.shape[:-1] + (k,)
    return np.array(vals, dtype=np.float32).reshape(shape), np.array(inds, dtype=np.int64).reshape(shape)
