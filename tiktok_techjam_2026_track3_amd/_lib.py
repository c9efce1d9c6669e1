"""ctypes binding of libmi355attn.so (the C-ABI declared in include/mi355attn.h).

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7`` dependency binds
to the HIP runtime torch already loaded (same SONAME): streams and device pointers from torch
are then valid handles for the library. There is no fallback: if the library is missing,
``lib()`` raises.
"""
from __future__ import annotations

import ctypes as C
import threading

import torch  # noqa: F401  (must precede the library load, see module docstring)

from .build import LIB_PATH

F32, F16, BF16 = 0, 1, 2

_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

# name -> (restype, argtypes); mirrors include/mi355attn.h
_P = C.c_void_p
_I64 = C.c_int64
_SIGNATURES = {
    "mi355_version": (C.c_int, []),
    "mi355_status_string": (C.c_char_p, [C.c_int]),
    "mi355_gemm_bias": (
        C.c_int,
        [C.c_int, C.c_int, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P],
    ),
    "mi355_attn_fwd": (
        C.c_int,
        [C.c_int, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
         C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64),
         C.c_float, C.c_int, _P, _I64, _P],
    ),
    "mi355_attn_workspace_bytes": (_I64, [C.c_int, _I64, _I64, _I64, _I64, _I64]),
    "mi355_attn_workspace_bytes_forced": (_I64, [C.c_int, _I64, _I64, _I64, _I64, _I64]),
    "mi355_attn_fwd_ws": (
        C.c_int,
        [C.c_int, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
         C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64),
         C.c_float, C.c_int, _P, _I64, _P, _I64, _P],
    ),
    "mi355_attn_fwd_kb": (
        C.c_int,
        [C.c_int, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
         C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64),
         C.c_float, C.c_int, _P, _I64, _P, _I64, C.c_int, _I64, _P],
    ),
    "mi355_gemm_bias_kbound": (
        C.c_int,
        [C.c_int, C.c_int, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64,
         _P, _I64, _I64, _I64, _I64, _P, _P],
    ),
    "mi355_layernorm_gemm_bias_kbound": (
        C.c_int,
        [C.c_int, C.c_int, _P, _I64, _P, _I64, _P, _P, C.c_float, _P, _P, _I64, _I64, _I64, _I64,
         _P, _I64, _I64, _I64, _I64, _P, _P],
    ),
    "mi355_quant_rows_i8": (C.c_int, [C.c_int, _P, _I64, _P, _P, _I64, _I64, C.c_int, _P]),
    "mi355_layernorm": (C.c_int, [C.c_int, _P, _I64, _P, _P, C.c_float, _P, _I64, _I64, _I64, _P]),
    "mi355_layernorm_cvt": (
        C.c_int, [C.c_int, C.c_int, _P, _I64, _P, _P, C.c_float, _P, _I64, _I64, _I64, _P],
    ),
    "mi355_gemm_bias_residual": (
        C.c_int,
        [C.c_int, C.c_int, _P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _P],
    ),
    "mi355_gemm_bias_gelu": (
        C.c_int, [C.c_int, C.c_int, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P],
    ),
    "mi355_gemm_bias_residual_zero_masked": (
        C.c_int,
        [C.c_int, C.c_int, _P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _P],
    ),
    "mi355_layernorm_masked": (
        C.c_int, [C.c_int, _P, _I64, _P, _P, C.c_float, _P, _I64, _I64, _I64, _P, _P],
    ),
    "mi355_gemm_i8": (
        C.c_int,
        [_P, _P, _P, _P, _P, C.c_int, _P, _I64, _P, _I64, _I64, _I64, _P, _P],
    ),
    "mi355_layernorm_gemm_bias": (
        C.c_int,
        [C.c_int, C.c_int, _P, _I64, _P, _I64, _P, _P, C.c_float, _P, _P, _I64, _I64, _I64, _I64,
         C.c_int, _P],
    ),
    "mi355_layernorm_gemm_bias_noalloc": (
        C.c_int,
        [C.c_int, C.c_int, _P, _I64, _P, _I64, _P, _P, C.c_float, _P, _I64, _I64, _I64, _I64,
         C.c_int, _P],
    ),
    "mi355_gemm_i8_epilogue": (
        C.c_int,
        [_P, _P, _P, _P, _P, C.c_int, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, C.c_int, _P],
    ),
}

# epilogue flags of mi355_gemm_i8_epilogue (MI355_EPI_*)
EPI_GELU = 1
EPI_ZERO_MASKED = 2

EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_handle: C.CDLL | None = None


class KernelError(RuntimeError):
    """A libmi355attn entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.fn = fn
        self.status = status


def lib() -> C.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _handle
    if _handle is not None:
        return _handle
    with _lock:
        if _handle is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with "
                    "`python -m tiktok_techjam_2026_track3_amd.build` (no fallback path exists)"
                )
            h = C.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _handle = h
    return _handle


def status_string(status: int) -> str:
    return lib().mi355_status_string(int(status)).decode()


def check(fn: str, status: int) -> None:
    if status != 0:
        raise KernelError(fn, status, status_string(status))


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def i64_array(values) -> "C.Array":
    vals = [int(v) for v in values]
    return (_I64 * len(vals))(*vals)
