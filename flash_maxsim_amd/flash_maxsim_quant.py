"""Per-token uint8 quantisation and the fused dequant MaxSim on MI355X.

Mirrors the reference module flash_maxsim/flash_maxsim_quant.py:
quantize_int8 (:11-28), dequantize_int8 (:31-33) and flash_maxsim_int8
(:105-142), with the same names, defaults, shapes and casts.

flash_maxsim_int8 runs libflashmaxsim's uint8 kernels. Queries of up to 64
tokens (and d > 256, and d > 128 over docs longer than 128 tokens) widen codes to
fp16 exactly in registers and apply the per-token affine map to the fp32 MFMA
result, S = scale * (Q . codes) + min * sum(Q), which equals Q . dequantize(codes)
up to fp32 rounding. Longer queries at d <= 128, and over docs of up to 128
tokens at d <= 256, dequantise each code to fp16 (code * scale + min, rounded
once) before the dot product, as the reference's kernel does; the two differ by
under 1e-3 per score.
"""

from __future__ import annotations

import torch

from . import _lib
from .flash_maxsim import _check_devices, _device_guard, _lengths, _prep


def quantize_int8(D: torch.Tensor):
    """Encodes every doc token as 8-bit codes on its own affine grid.

    For the d values x of one token, lo = min(x), step = max((max(x) - lo) / 255,
    1e-8) in float32, and code = clamp(round_half_even((x - lo) / step), 0, 255).
    Returns (codes uint8 [B, Ld, d], step fp16 [B, Ld, 1], lo fp16 [B, Ld, 1]):
    codes come from the float32 step, the stored step and lo are rounded to
    fp16 - the storage format flash_maxsim_int8 reads (reference
    flash_maxsim_quant.py:11-28, whose arithmetic this matches bit for bit).
    """
    assert D.dim() == 3
    if D.is_cuda:
        return _quantize_gpu(D)
    x = D.to(torch.float32)
    lo, hi = torch.aminmax(x, dim=-1, keepdim=True)
    step = torch.clamp_min((hi - lo) / 255.0, 1e-8)
    codes = torch.clamp(torch.round((x - lo) / step), 0, 255).to(torch.uint8)
    return codes, step.to(torch.float16), lo.to(torch.float16)


_SRC_CODES = {torch.float16: _lib.FMX_DTYPE_F16, torch.bfloat16: _lib.FMX_DTYPE_BF16,
              torch.float32: _lib.FMX_DTYPE_F32}


def _quant_source(D: torch.Tensor) -> torch.Tensor:
    """D as fp16/bf16/fp32 with unit inner stride (other dtypes go through fp32,
    as the torch formula's D.to(float32) does)."""
    if D.dtype not in _SRC_CODES:
        D = D.to(torch.float32)
    if D.stride(-1) != 1 or (D.dim() == 3 and D.shape[1] > 1 and D.stride(1) < D.shape[2]):
        D = D.contiguous()
    return D


def _quantize_gpu(D: torch.Tensor):
    """quantize_int8 in one pass of libflashmaxsim's HIP encoder; bit-identical
    to the torch formula (same IEEE fp32 operations, same order)."""
    B, Ld, d = D.shape
    src = _quant_source(D)
    dev = _check_devices(src)
    codes = torch.empty(B, Ld, d, device=dev, dtype=torch.uint8)
    scales = torch.empty(B, Ld, 1, device=dev, dtype=torch.float16)
    mins = torch.empty(B, Ld, 1, device=dev, dtype=torch.float16)
    if B == 0 or Ld == 0 or d == 0:
        if d == 0:  # empty rows: min/max of nothing, as torch.aminmax raises
            raise RuntimeError("quantize_int8 needs d >= 1")
        return codes, scales, mins
    lib = _lib.load()
    with _device_guard(dev):
        rc = lib.fmx_quantize_int8(
            _SRC_CODES[src.dtype], src.data_ptr(), src.stride(0), src.stride(1), B, Ld, d, None, None, 0,
            codes.data_ptr(), d, scales.data_ptr(), mins.data_ptr(), Ld, _lib.stream_of(src),
        )
    _lib.check(rc)
    return codes, scales, mins


def dequantize_int8(D_uint8: torch.Tensor, scales: torch.Tensor, mins: torch.Tensor) -> torch.Tensor:
    """float32 doc tokens back from codes: code * step + lo (reference
    flash_maxsim_quant.py:31-33; a separate multiply and add, no fma)."""
    return D_uint8.to(torch.float32) * scales.to(torch.float32) + mins.to(torch.float32)


def _scale_rows(t: torch.Tensor, Ld: int) -> torch.Tensor:
    """fp16 [B, Ld] scale or min rows as the kernels read them: t itself when
    its tokens are adjacent and its rows at least Ld apart (any 2-byte
    alignment), else a contiguous fp16 copy (reference :129-130 copies always)."""
    if t.dtype == torch.float16 and t.stride(-1) == 1 and t.stride(0) >= Ld:
        return t
    return t.contiguous().half()


def flash_maxsim_int8(
    Q: torch.Tensor,
    D_uint8: torch.Tensor,
    scales: torch.Tensor,
    mins: torch.Tensor,
    doc_lengths=None,
) -> torch.Tensor:
    """flash_maxsim over quantize_int8-encoded docs: float32 [B].

    Q is [Lq, d]; D_uint8 [B, Ld, d] uint8 codes with per-token scales and mins
    of shape [B, Ld, 1] or [B, Ld]. Reference signature:
    flash_maxsim_quant.py:105.
    """
    assert Q.dim() == 2 and D_uint8.dim() == 3 and Q.shape[1] == D_uint8.shape[2]
    Lq, d = Q.shape
    B, Ld, _ = D_uint8.shape
    if D_uint8.dtype != torch.uint8:
        raise TypeError(f"D_uint8 must be torch.uint8, got {D_uint8.dtype}")

    if scales.dim() == 3:
        scales = scales.squeeze(-1)
    if mins.dim() == 3:
        mins = mins.squeeze(-1)
    assert tuple(scales.shape) == (B, Ld) and tuple(mins.shape) == (B, Ld), "scales/mins must be [B, Ld(, 1)]"

    lengths = _lengths(B, D_uint8.device, doc_lengths)
    Q = _prep(Q, torch.float16)
    D_uint8 = _prep(D_uint8, None)
    scales, mins = _scale_rows(scales, Ld), _scale_rows(mins, Ld)
    if scales.stride(0) != mins.stride(0):  # the kernel takes one row stride for both
        scales, mins = scales.contiguous(), mins.contiguous()
    dev = _check_devices(Q, D_uint8, scales, mins, lengths)
    scores = torch.empty(B, device=dev, dtype=torch.float32)
    if B == 0:
        return scores
    if Lq == 0:
        return scores.zero_()

    lib = _lib.load()
    nbytes = lib.fmx_fwd_int8_workspace_bytes(B, Lq, Ld, d)
    ws = _lib.workspace(nbytes, dev)
    with _device_guard(dev):
        rc = lib.fmx_fwd_int8(
            Q.data_ptr(), Q.stride(0), D_uint8.data_ptr(), D_uint8.stride(0), D_uint8.stride(1),
            scales.data_ptr(), mins.data_ptr(), scales.stride(0), _lib.ptr(lengths), scores.data_ptr(),
            B, Lq, Ld, d, _lib.ptr(ws), nbytes, _lib.stream_of(Q),
        )
    _lib.check(rc)
    return scores
