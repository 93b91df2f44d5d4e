"""ctypes binding of libflashmaxsim.so (declarations in include/fmx.h).

torch is imported first so the HIP runtime bundled with torch is already
loaded: libflashmaxsim's libamdhip64.so.7 dependency then resolves to that same
runtime, and torch's streams and device pointers are valid inside the library.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must load the HIP runtime before the library)

LIB_PATH = Path(__file__).resolve().with_name("libflashmaxsim.so")

FMX_DTYPE_F16 = 0
FMX_DTYPE_BF16 = 1
FMX_DTYPE_F32 = 2

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p
_int = ctypes.c_int
_size = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGNATURES = {
    "fmx_version": (ctypes.c_char_p, []),
    "fmx_last_error": (ctypes.c_char_p, []),
    "fmx_fwd": (
        _int,
        [_int, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _ptr,
         _i64, _i64, _i64, _i64, _i64, _int, _ptr, _size, _ptr],
    ),
    "fmx_fwd_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "fmx_fwd_noalloc": (
        _int,
        [_int, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _ptr,
         _i64, _i64, _i64, _i64, _i64, _int, _ptr],
    ),
    "fmx_fwd_int8": (
        _int,
        [_ptr, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _ptr, _ptr,
         _i64, _i64, _i64, _i64, _ptr, _size, _ptr],
    ),
    "fmx_fwd_int8_workspace_bytes": (_size, [_i64, _i64, _i64, _i64]),
    "fmx_fwd_sparse": (
        _int,
        [_int, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _ptr,
         _i64, _i64, _i64, _ptr, _size, _ptr],
    ),
    "fmx_fwd_sparse_workspace_bytes": (_size, [_i64, _i64, _i64, _i64]),
    "fmx_quantize_int8": (
        _int,
        [_int, _ptr, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _i64, _ptr, _ptr, _i64, _ptr],
    ),
    "fmx_fwd_packed": (
        _int,
        [_int, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _ptr, _size, _ptr],
    ),
    "fmx_fwd_packed_workspace_bytes": (_size, [_i64, _i64, _i64, _i64]),
    "fmx_fwd_int8_packed": (
        _int,
        [_ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _ptr, _size, _ptr],
    ),
    "fmx_fwd_int8_packed_workspace_bytes": (_size, [_i64, _i64, _i64, _i64]),
    "fmx_topk": (_int, [_ptr, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _size, _ptr]),
    "fmx_topk_workspace_bytes": (_size, [_i64, _i64, _i64]),
    "fmx_fwd_topk": (
        _int,
        [_int, _ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _size,
         _ptr],
    ),
    "fmx_fwd_topk_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "fmx_bwd": (
        _int,
        [_int, _ptr, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr, _ptr,
         _i64, _i64, _i64, _i64, _ptr, _size, _ptr],
    ),
    "fmx_bwd_workspace_bytes": (_size, [_i64, _i64, _i64, _i64]),
    "fmx_bwd_batched": (
        _int,
        [_int, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _ptr,
         _i64, _i64, _i64, _i64, _i64, _ptr, _size, _ptr],
    ),
    "fmx_bwd_batched_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64]),
}

EXPORTED = tuple(_SIGNATURES)

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Loads libflashmaxsim.so once; raises if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP extension first "
                "(`python -m flash_maxsim_amd.build`, needs hipcc for gfx950)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().fmx_last_error().decode(errors="replace")
        raise RuntimeError(f"flash_maxsim_amd: {msg} (code {rc})")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return FMX_DTYPE_F16
    if t.dtype == torch.bfloat16:
        return FMX_DTYPE_BF16
    raise TypeError(f"kernel operands must be float16 or bfloat16, got {t.dtype}")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)
