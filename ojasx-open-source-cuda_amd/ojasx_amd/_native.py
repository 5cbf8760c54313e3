"""Loader for libojasx_e8t.so, the HIP kernels behind the C ABI in include/ojasx_e8t.h.

There is no fallback: if the library is missing or the tensors are not on a
ROCm device, every op raises.  The library is loaded with ctypes so that the
product depends only on the HIP runtime and torch's public Python API.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_ROOT, "lib", "libojasx_e8t.so")

F32, F16, BF16, F64 = 0, 1, 2, 3
DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

EXPORTS = (
    "ojx_e8t_version",
    "ojx_e8t_last_error",
    "ojx_e8t_encode",
    "ojx_e8t_decode",
    "ojx_gemm_workspace_bytes",
    "ojx_e8t_gemm_fwd",
    "ojx_e8t_gemm_fwd_noalloc",
    "ojx_lora_down",
    "ojx_e8t_gemm_fwd_lora",
    "ojx_e8_gemm_fwd_lora",
    "ojx_e8r_gemm_fwd_lora",
    "ojx_e8t_gemm_bwd_dx",
    "ojx_e8t_gemv_grouped_plan",
    "ojx_e8t_gemv_grouped",
    "ojx_e8_gemv_grouped_plan",
    "ojx_e8_gemv_grouped",
    "ojx_e8r_gemv_grouped_plan",
    "ojx_e8r_gemv_grouped",
    "ojx_e8_encode",
    "ojx_e8_decode",
    "ojx_e8_gemm_fwd",
    "ojx_e8_gemm_bwd_dx",
    "ojx_e8r_encode",
    "ojx_e8r_decode",
    "ojx_e8r_gemm_fwd",
    "ojx_e8r_gemm_bwd_dx",
    "ojx_fwht32",
    "ojx_e8_cs_project",
    "ojx_e8_ste_quantize",
    "ojx_e8_cs_project_dt",
    "ojx_e8_ste_quantize_dt",
)


class GemvJob(ctypes.Structure):
    """ojx_e8t_gemv_job of include/ojasx_e8t.h."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("packed", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("N", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("y_col", ctypes.c_int64),
        ("y_ld", ctypes.c_int64),
        ("wg_begin", ctypes.c_int64),
        ("lora_u", ctypes.c_void_p),
        ("lora_b", ctypes.c_void_p),
        ("lora_r", ctypes.c_int64),
        ("lora_ldu", ctypes.c_int64),
        ("lora_a", ctypes.c_void_p),
        ("lora_scaling", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]

_lib = None
_lock = threading.Lock()

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_SZ = ctypes.c_size_t
_F32 = ctypes.c_float


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"ojasx_amd: {LIB_PATH} is missing; build it with "
                    "`python ojasx-open-source-cuda_amd/build.py` (hipcc, gfx950)")
            L = ctypes.CDLL(LIB_PATH)
            L.ojx_e8t_version.restype = _INT
            L.ojx_e8t_version.argtypes = []
            L.ojx_e8t_last_error.restype = ctypes.c_char_p
            L.ojx_e8t_last_error.argtypes = []
            L.ojx_e8t_encode.restype = _INT
            L.ojx_e8t_encode.argtypes = [_P, _INT, _I64, _I64, _P, _P, _P]
            L.ojx_e8t_decode.restype = _INT
            L.ojx_e8t_decode.argtypes = [_P, _P, _I64, _I64, _INT, _P, _P]
            L.ojx_gemm_workspace_bytes.restype = _INT
            L.ojx_gemm_workspace_bytes.argtypes = [_INT, _INT, _I64, _I64, _I64, _I64, _INT, _P]
            L.ojx_e8t_gemm_fwd.restype = _INT
            L.ojx_e8t_gemm_fwd.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P,
                                          _SZ, _P]
            L.ojx_e8t_gemm_fwd_noalloc.restype = _INT
            L.ojx_e8t_gemm_fwd_noalloc.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                                   _INT, _P]
            L.ojx_lora_down.restype = _INT
            L.ojx_lora_down.argtypes = [_P, _P, _I64, _I64, _I64, _F32, _INT, _P, _P]
            for name in ("ojx_e8t_gemm_fwd_lora", "ojx_e8_gemm_fwd_lora", "ojx_e8r_gemm_fwd_lora"):
                fn = getattr(L, name)
                fn.restype = _INT
                fn.argtypes = [_P, _P, _P, _P, _P, _P, _I64, _F32, _P, _P, _I64, _I64, _I64,
                               _I64, _INT, _P, _SZ, _P]
            L.ojx_e8t_gemm_bwd_dx.restype = _INT
            L.ojx_e8t_gemm_bwd_dx.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P,
                                             _SZ, _P]
            L.ojx_e8t_gemv_grouped_plan.restype = _INT
            L.ojx_e8t_gemv_grouped_plan.argtypes = [_P, _INT, _I64, _INT, _P]
            L.ojx_e8t_gemv_grouped.restype = _INT
            L.ojx_e8t_gemv_grouped.argtypes = [_P, _P, _INT, _P, _P, _I64, _INT, _P]
            L.ojx_e8_gemv_grouped_plan.restype = _INT
            L.ojx_e8_gemv_grouped_plan.argtypes = [_P, _INT, _I64, _I64, _INT, _P]
            L.ojx_e8_gemv_grouped.restype = _INT
            L.ojx_e8_gemv_grouped.argtypes = [_P, _P, _INT, _P, _P, _I64, _I64, _INT, _P]
            L.ojx_e8r_gemv_grouped_plan.restype = _INT
            L.ojx_e8r_gemv_grouped_plan.argtypes = [_P, _INT, _I64, _I64, _INT, _P]
            L.ojx_e8r_gemv_grouped.restype = _INT
            L.ojx_e8r_gemv_grouped.argtypes = [_P, _P, _INT, _P, _P, _I64, _I64, _INT, _P]
            L.ojx_e8_encode.restype = _INT
            L.ojx_e8_encode.argtypes = [_P, _INT, _I64, _I64, _P, _P, _P]
            L.ojx_e8_decode.restype = _INT
            L.ojx_e8_decode.argtypes = [_P, _P, _I64, _I64, _INT, _P, _P]
            L.ojx_e8_gemm_fwd.restype = _INT
            L.ojx_e8_gemm_fwd.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P,
                                          _SZ, _P]
            L.ojx_e8_gemm_bwd_dx.restype = _INT
            L.ojx_e8_gemm_bwd_dx.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P,
                                             _SZ, _P]
            L.ojx_e8r_encode.restype = _INT
            L.ojx_e8r_encode.argtypes = [_P, _INT, _I64, _I64, _P, _P, _P]
            L.ojx_e8r_decode.restype = _INT
            L.ojx_e8r_decode.argtypes = [_P, _P, _I64, _I64, _INT, _P, _P]
            L.ojx_e8r_gemm_fwd.restype = _INT
            L.ojx_e8r_gemm_fwd.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P,
                                          _SZ, _P]
            L.ojx_e8r_gemm_bwd_dx.restype = _INT
            L.ojx_e8r_gemm_bwd_dx.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P,
                                             _SZ, _P]
            L.ojx_fwht32.restype = _INT
            L.ojx_fwht32.argtypes = [_P, _INT, _I64, _P, _P]
            L.ojx_e8_cs_project.restype = _INT
            L.ojx_e8_cs_project.argtypes = [_P, _INT, _I64, _P, _P]
            L.ojx_e8_ste_quantize.restype = _INT
            L.ojx_e8_ste_quantize.argtypes = [_P, _I64, _P, _P]
            L.ojx_e8_cs_project_dt.restype = _INT
            L.ojx_e8_cs_project_dt.argtypes = [_P, _INT, _I64, _P, _P]
            L.ojx_e8_ste_quantize_dt.restype = _INT
            L.ojx_e8_ste_quantize_dt.argtypes = [_P, _INT, _I64, _P, _P]
            _lib = L
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().ojx_e8t_last_error().decode(errors="replace")
        raise RuntimeError(f"ojasx_e8t {what} failed (status {status}): {msg}")


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "ojasx_amd E8 kernels run on ROCm devices only (got a tensor on "
                f"{t.device}); move the layer / tensors to the GPU")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
