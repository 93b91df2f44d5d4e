"""Per-token uint8 quantisation and the fused dequant MaxSim on MI355X.

Mirrors the reference module flash_maxsim/flash_maxsim_quant.py:
quantize_int8 (:11-28), dequantize_int8 (:31-33) and flash_maxsim_int8
(:105-142), with the same names, defaults, shapes and casts.

flash_maxsim_int8 runs libflashmaxsim's uint8 kernel: codes are widened to fp16
exactly in registers and the per-token affine map is applied to the fp32 MFMA
result, S = scale * (Q . codes) + min * sum(Q), which equals Q . dequantize(codes)
up to fp32 rounding. (The reference dequantises in fp16 before its dot product.)
"""

from __future__ import annotations

import torch

from . import _lib
from .flash_maxsim import _check_devices, _device_guard, _lengths, _prep


def quantize_int8(D: torch.Tensor):
    """Per-token affine INT8 quantization.

    Args:
        D: [B, Ld, d] float/half tensor.

    Returns:
        D_uint8: [B, Ld, d] uint8
        scales:  [B, Ld, 1] float16
        mins:    [B, Ld, 1] float16
    """
    assert D.dim() == 3
    Df = D.float()
    d_min = Df.min(dim=-1, keepdim=True).values
    d_max = Df.max(dim=-1, keepdim=True).values
    scales = ((d_max - d_min) / 255.0).clamp_min(1e-8)
    D_uint8 = ((Df - d_min) / scales).round().clamp(0, 255).to(torch.uint8)
    return D_uint8, scales.half(), d_min.half()


def dequantize_int8(D_uint8: torch.Tensor, scales: torch.Tensor, mins: torch.Tensor) -> torch.Tensor:
    """Reconstruct float tensors from per-token affine INT8 encoding."""
    return D_uint8.float() * scales.float() + mins.float()


def flash_maxsim_int8(
    Q: torch.Tensor,
    D_uint8: torch.Tensor,
    scales: torch.Tensor,
    mins: torch.Tensor,
    doc_lengths=None,
) -> torch.Tensor:
    """Fused dequant+MaxSim. Q: [Lq, d], D_uint8: [B, Ld, d] -> [B]."""
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
    scales = scales.contiguous().half()
    mins = mins.contiguous().half()
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
