"""CPU oracle for the E8 quantized-weight paths (ternary 1.5-bit and 2-bit) -- TEST
INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this module, and only as the checker.  The product package never
imports it.

Two native checkers are wrapped here:

* ``lib/libojx_oracle.so`` -- this repository's C restatement of the
  reference's codec (``e8t_oracle.c``; ``ojasx2/math/lattice.py:286-419``).
* ``_ref/libojx_refcore.so`` -- the reference's own header-only C++ kernels
  (``ojasx2/math/csrc/ojasx_math_core.hpp:549-702``) compiled from the
  reference sources by ``oracle/Makefile``.  Optional: ``ref_available()``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "lib", "libojx_oracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libojx_refcore.so")

_lib = None
_ref = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def build() -> None:
    """Compile the oracle (and the reference checker when the reference is present)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.ojo_f32_to_f16.restype = ctypes.c_uint16
        L.ojo_f32_to_f16.argtypes = [ctypes.c_float]
        L.ojo_f32_to_bf16.restype = ctypes.c_uint16
        L.ojo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.ojo_f16_to_f32.restype = ctypes.c_float
        L.ojo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.ojo_e8t_group_scale.restype = ctypes.c_float
        L.ojo_e8t_group_scale.argtypes = [_P, _I64]
        L.ojo_e8t_quantize8.restype = ctypes.c_int32
        L.ojo_e8t_quantize8.argtypes = [_P, _P]
        L.ojo_e8t_codeword.restype = None
        L.ojo_e8t_codeword.argtypes = [ctypes.c_int32, _P]
        L.ojo_e8t_padded.restype = _I64
        L.ojo_e8t_padded.argtypes = [_I64, _I64]
        L.ojo_e8t_effective_gs.restype = _I64
        L.ojo_e8t_effective_gs.argtypes = [_I64]
        L.ojo_e8t_encode.restype = None
        L.ojo_e8t_encode.argtypes = [_P, _I64, _I64, _P, _P, _P, ctypes.c_int]
        L.ojo_e8t_decode.restype = None
        L.ojo_e8t_decode.argtypes = [_P, _P, _I64, _I64, ctypes.c_int, _P]
        L.ojo_e8t_gemm_f64.restype = None
        L.ojo_e8t_gemm_f64.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_int]
        L.ojo_e8t_gemm_bwd_f64.restype = None
        L.ojo_e8t_gemm_bwd_f64.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_int]
        for name in ("ojo_f32_to_f16_array", "ojo_f32_to_bf16_array"):
            getattr(L, name).restype = None
            getattr(L, name).argtypes = [_P, _P, _I64]
        L.ojo_e8t_group_scale_array.restype = None
        L.ojo_e8t_group_scale_array.argtypes = [_P, _I64, _I64, _P]
        L.ojo_e8t_quantize8_array.restype = None
        L.ojo_e8t_quantize8_array.argtypes = [_P, _I64, _P]
        L.ojo_e8b_check_gs.restype = _I64
        L.ojo_e8b_check_gs.argtypes = [_I64]
        L.ojo_e8b_quantize8.restype = None
        L.ojo_e8b_quantize8.argtypes = [_P, _P]
        L.ojo_e8b_quantize8_array.restype = None
        L.ojo_e8b_quantize8_array.argtypes = [_P, _I64, _P]
        L.ojo_e8b_encode.restype = None
        L.ojo_e8b_encode.argtypes = [_P, _I64, _I64, _P, _P, _P, ctypes.c_int]
        L.ojo_e8b_decode.restype = None
        L.ojo_e8b_decode.argtypes = [_P, _P, _I64, _I64, ctypes.c_int, _P]
        L.ojo_e8b_gemm_f64.restype = None
        L.ojo_e8b_gemm_f64.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_int]
        L.ojo_e8b_gemm_bwd_f64.restype = None
        L.ojo_e8b_gemm_bwd_f64.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_int]
        L.ojo_e8r_lut.restype = None
        L.ojo_e8r_lut.argtypes = [_P]
        L.ojo_e8r_quantize8.restype = ctypes.c_int32
        L.ojo_e8r_quantize8.argtypes = [_P]
        L.ojo_e8r_quantize8_array.restype = None
        L.ojo_e8r_quantize8_array.argtypes = [_P, _I64, _P]
        L.ojo_e8r_row_sum.restype = ctypes.c_float
        L.ojo_e8r_row_sum.argtypes = [_P, _I64]
        L.ojo_e8r_encode.restype = None
        L.ojo_e8r_encode.argtypes = [_P, _I64, _I64, _P, _P, _P, ctypes.c_int]
        L.ojo_e8r_decode.restype = None
        L.ojo_e8r_decode.argtypes = [_P, _P, _I64, _I64, ctypes.c_int, _P]
        L.ojo_e8r_gemm_f64.restype = None
        L.ojo_e8r_gemm_f64.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_int]
        L.ojo_e8r_gemm_bwd_f64.restype = None
        L.ojo_e8r_gemm_bwd_f64.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_int]
        L.ojo_e8_cs_project_f32.restype = None
        L.ojo_e8_cs_project_f32.argtypes = [_P, _P, _I64]
        L.ojo_e8_cs_project_f64.restype = None
        L.ojo_e8_cs_project_f64.argtypes = [_P, _P, _I64]
        L.ojo_e8_ste_quantize_f32.restype = None
        L.ojo_e8_ste_quantize_f32.argtypes = [_P, _I64, _P]
        L.ojo_e8_cs_project_half.restype = None
        L.ojo_e8_cs_project_half.argtypes = [_P, _P, _I64, ctypes.c_int]
        L.ojo_e8_ste_quantize_half.restype = None
        L.ojo_e8_ste_quantize_half.argtypes = [_P, _I64, _P, ctypes.c_int]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(_REF_PATH)


def ref() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        R = ctypes.CDLL(_REF_PATH)
        R.ojr_ternary_lut.restype = ctypes.POINTER(ctypes.c_int8)
        R.ojr_ternary_lut.argtypes = []
        R.ojr_ternary_fwd_f32.restype = None
        R.ojr_ternary_fwd_f32.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]
        R.ojr_ternary_bwd_dx_f32.restype = None
        R.ojr_ternary_bwd_dx_f32.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64]
        R.ojr_e8_fwd_f32.restype = None
        R.ojr_e8_fwd_f32.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]
        R.ojr_e8_bwd_dx_f32.restype = None
        R.ojr_e8_bwd_dx_f32.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64]
        _ref = R
    return _ref


# --------------------------------------------------------------------------
# dtype codes shared with the product's C ABI: 0 fp32, 1 fp16, 2 bf16
# --------------------------------------------------------------------------
DT_F32, DT_F16, DT_BF16 = 0, 1, 2


def f32_to_f16_bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().ojo_f32_to_f16_array(_ptr(a), _ptr(out), a.size)
    return out


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().ojo_f32_to_bf16_array(_ptr(a), _ptr(out), a.size)
    return out


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def effective_gs(gs: int) -> int:
    return int(lib().ojo_e8t_effective_gs(int(gs)))


def padded(numel: int, gs: int) -> int:
    return int(lib().ojo_e8t_padded(int(numel), int(gs)))


def group_scales(w_groups: np.ndarray) -> np.ndarray:
    """fp32 scale of each row of ``w_groups`` ([G, gs] fp32)."""
    w = np.ascontiguousarray(w_groups, dtype=np.float32)
    G, gs = w.shape
    out = np.empty(G, dtype=np.float32)
    lib().ojo_e8t_group_scale_array(_ptr(w), G, gs, _ptr(out))
    return out


def quantize8(v: np.ndarray) -> Tuple[int, np.ndarray]:
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(8)
    q = np.empty(8, dtype=np.int8)
    code = lib().ojo_e8t_quantize8(_ptr(v), _ptr(q))
    return int(code), q


def quantize8_many(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1, 8)
    out = np.empty(v.shape[0], dtype=np.int32)
    lib().ojo_e8t_quantize8_array(_ptr(v), v.shape[0], _ptr(out))
    return out


def codeword(code: int) -> np.ndarray:
    c = np.empty(8, dtype=np.int8)
    lib().ojo_e8t_codeword(int(code), _ptr(c))
    return c


def codebook() -> np.ndarray:
    """[3281, 8] int8 coordinates in rank order (closed form raw = 2 * rank)."""
    return np.stack([codeword(c) for c in range(3281)])


def encode(w: np.ndarray, group_size: int = 32, nthreads: int = 0
           ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """TernaryE8LatticePacker.pack on the flattened fp32 values of ``w``.

    Returns (packed uint8 [padded*3/16], scales fp16 bits uint16 [padded/gs],
    scales32 fp32 [padded/gs])."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    gs = effective_gs(group_size)
    p = padded(w.size, gs)
    packed = np.empty(p * 3 // 16, dtype=np.uint8)
    scales = np.empty(p // gs, dtype=np.uint16)
    scales32 = np.empty(p // gs, dtype=np.float32)
    lib().ojo_e8t_encode(_ptr(w), w.size, gs, _ptr(packed), _ptr(scales), _ptr(scales32),
                         int(nthreads))
    return packed, scales, scales32


def unpack_codes(packed: np.ndarray) -> np.ndarray:
    """Bytes -> 12-bit codes (lattice.py:397-405), vectorised closed form."""
    t = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1, 3).astype(np.int32)
    c0 = t[:, 0] | ((t[:, 1] & 0x0F) << 8)
    c1 = ((t[:, 1] >> 4) & 0x0F) | (t[:, 2] << 4)
    return np.stack([c0, c1], axis=1).reshape(-1)


def decode(packed: np.ndarray, scales: np.ndarray, numel: int, group_size: int,
           dtype: int = DT_F32) -> np.ndarray:
    """TernaryE8LatticePacker.unpack: fp32 values, or fp16 / bf16 bit patterns."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    out = np.empty(numel, dtype=np.float32 if dtype == DT_F32 else np.uint16)
    lib().ojo_e8t_decode(_ptr(packed), _ptr(scales), numel, int(group_size), int(dtype),
                         _ptr(out))
    return out


def gemm_f64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray,
             bias: Optional[np.ndarray], N: int, K: int, group_size: int,
             w_dtype: int = DT_F32) -> np.ndarray:
    """fp64-accumulated x @ Wdeq^T + bias with Wdeq decoded per the dtype rule."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    M = x.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().ojo_e8t_gemm_f64(_ptr(x), _ptr(np.ascontiguousarray(packed)),
                           _ptr(np.ascontiguousarray(scales, dtype=np.uint16)),
                           None if b is None else _ptr(b), _ptr(y), M, N, K,
                           int(group_size), int(w_dtype))
    return y


def gemm_bwd_f64(gy: np.ndarray, packed: np.ndarray, scales: np.ndarray, N: int, K: int,
                 group_size: int, w_dtype: int = DT_F32) -> np.ndarray:
    gy = np.ascontiguousarray(gy, dtype=np.float32).reshape(-1, N)
    M = gy.shape[0]
    gx = np.empty((M, K), dtype=np.float64)
    lib().ojo_e8t_gemm_bwd_f64(_ptr(gy), _ptr(np.ascontiguousarray(packed)),
                               _ptr(np.ascontiguousarray(scales, dtype=np.uint16)), _ptr(gx),
                               M, N, K, int(group_size), int(w_dtype))
    return gx


# --------------------------------------------------------------------------
# The reference's own C++ kernels (oracle/_ref)
# --------------------------------------------------------------------------

def ref_codebook() -> np.ndarray:
    p = ref().ojr_ternary_lut()
    return np.ctypeslib.as_array(p, shape=(3281 * 8,)).reshape(3281, 8).copy()


def ref_fused_fwd(x: np.ndarray, packed: np.ndarray, scales_f32: np.ndarray,
                  bias: Optional[np.ndarray], N: int, K: int, group_size: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    M = x.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    s = np.ascontiguousarray(scales_f32, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    ref().ojr_ternary_fwd_f32(_ptr(x), _ptr(np.ascontiguousarray(packed)), _ptr(s),
                              None if b is None else _ptr(b), _ptr(y), M, K, N,
                              int(group_size))
    return y


def ref_fused_bwd_dx(gy: np.ndarray, packed: np.ndarray, scales_f32: np.ndarray, N: int,
                     K: int, group_size: int) -> np.ndarray:
    gy = np.ascontiguousarray(gy, dtype=np.float32).reshape(-1, N)
    M = gy.shape[0]
    gx = np.empty((M, K), dtype=np.float32)
    s = np.ascontiguousarray(scales_f32, dtype=np.float32)
    ref().ojr_ternary_bwd_dx_f32(_ptr(gy), _ptr(np.ascontiguousarray(packed)), _ptr(s),
                                 _ptr(gx), M, K, N, int(group_size))
    return gx


# --------------------------------------------------------------------------
# 2-bit E8 (E8LatticePacker, lattice.py:209-279)
# --------------------------------------------------------------------------

def e8b_quantize8_many(v: np.ndarray) -> np.ndarray:
    """Codes (0..3) of n 8-vectors v [n, 8] (already divided by their scale)."""
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1, 8)
    codes = np.empty(v.shape, dtype=np.uint8)
    lib().ojo_e8b_quantize8_array(_ptr(v), v.shape[0], _ptr(codes))
    return codes


def e8b_encode(w: np.ndarray, group_size: int = 8, nthreads: int = 0
               ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """E8LatticePacker.pack on the flattened fp32 values of ``w``.

    Returns (packed uint8 [padded/4], scales fp16 bits uint16 [padded/gs],
    scales32 fp32 [padded/gs]).  A group size that is not a positive multiple of 8
    raises ValueError, as lattice.py:220-221 does."""
    if lib().ojo_e8b_check_gs(int(group_size)) < 0:
        raise ValueError(f"group_size ({group_size}) must be a positive multiple of 8.")
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    p = padded(w.size, group_size)
    packed = np.empty(p // 4, dtype=np.uint8)
    scales = np.empty(p // group_size, dtype=np.uint16)
    scales32 = np.empty(p // group_size, dtype=np.float32)
    lib().ojo_e8b_encode(_ptr(w), w.size, int(group_size), _ptr(packed), _ptr(scales),
                         _ptr(scales32), int(nthreads))
    return packed, scales, scales32


def e8b_decode(packed: np.ndarray, scales: np.ndarray, numel: int, group_size: int,
               dtype: int = DT_F32) -> np.ndarray:
    """E8LatticePacker.unpack: fp32 values, or fp16 / bf16 bit patterns."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    out = np.empty(numel, dtype=np.float32 if dtype == DT_F32 else np.uint16)
    lib().ojo_e8b_decode(_ptr(packed), _ptr(scales), numel, int(group_size), int(dtype),
                         _ptr(out))
    return out


def e8b_gemm_f64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray,
                 bias: Optional[np.ndarray], N: int, K: int, group_size: int,
                 w_dtype: int = DT_F32) -> np.ndarray:
    """fp64-accumulated x @ Wdeq^T + bias, Wdeq by the 2-bit dtype rule."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    M = x.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().ojo_e8b_gemm_f64(_ptr(x), _ptr(np.ascontiguousarray(packed)),
                           _ptr(np.ascontiguousarray(scales, dtype=np.uint16)),
                           None if b is None else _ptr(b), _ptr(y), M, N, K,
                           int(group_size), int(w_dtype))
    return y


def e8b_gemm_bwd_f64(gy: np.ndarray, packed: np.ndarray, scales: np.ndarray, N: int, K: int,
                     group_size: int, w_dtype: int = DT_F32) -> np.ndarray:
    gy = np.ascontiguousarray(gy, dtype=np.float32).reshape(-1, N)
    M = gy.shape[0]
    gx = np.empty((M, K), dtype=np.float64)
    lib().ojo_e8b_gemm_bwd_f64(_ptr(gy), _ptr(np.ascontiguousarray(packed)),
                               _ptr(np.ascontiguousarray(scales, dtype=np.uint16)), _ptr(gx),
                               M, N, K, int(group_size), int(w_dtype))
    return gx


def ref_e8_fused_fwd(x: np.ndarray, packed: np.ndarray, scales_f32: np.ndarray,
                     bias: Optional[np.ndarray], N: int, K: int, group_size: int) -> np.ndarray:
    """The reference's C++ 2-bit fused forward (ojasx_math_core.hpp:440-483)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    M = x.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    s = np.ascontiguousarray(scales_f32, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    ref().ojr_e8_fwd_f32(_ptr(x), _ptr(np.ascontiguousarray(packed)), _ptr(s),
                         None if b is None else _ptr(b), _ptr(y), M, K, N, int(group_size))
    return y


def ref_e8_fused_bwd_dx(gy: np.ndarray, packed: np.ndarray, scales_f32: np.ndarray, N: int,
                        K: int, group_size: int) -> np.ndarray:
    """The reference's C++ 2-bit fused backward dX (ojasx_math_core.hpp:490-534)."""
    gy = np.ascontiguousarray(gy, dtype=np.float32).reshape(-1, N)
    M = gy.shape[0]
    gx = np.empty((M, K), dtype=np.float32)
    s = np.ascontiguousarray(scales_f32, dtype=np.float32)
    ref().ojr_e8_bwd_dx_f32(_ptr(gy), _ptr(np.ascontiguousarray(packed)), _ptr(s), _ptr(gx),
                            M, K, N, int(group_size))
    return gx


# --------------------------------------------------------------------------- 1-bit Root E8

def e8r_effective_gs(gs: int) -> int:
    """RootE8LatticePacker.pack's silent coercion (lattice.py:485-486)."""
    return 8 if (gs <= 0 or gs % 8 != 0) else int(gs)


def e8r_lut() -> np.ndarray:
    """The 256 x 8 table of lattice.py:436-456 (x2), fp32."""
    out = np.empty(256 * 8, dtype=np.float32)
    lib().ojo_e8r_lut(_ptr(out))
    return out.reshape(256, 8)


def e8r_quantize8_many(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1, 8)
    codes = np.empty(v.shape[0], dtype=np.int32)
    lib().ojo_e8r_quantize8_array(_ptr(v), v.shape[0], _ptr(codes))
    return codes


def e8r_row_sum(x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    return float(lib().ojo_e8r_row_sum(_ptr(x), x.size))


def e8r_encode(w: np.ndarray, group_size: int = 32, nthreads: int = 0
               ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """RootE8LatticePacker.pack on the flattened fp32 values of ``w``.

    Returns (codes uint8 [padded/8], scales fp16 bits uint16 [padded/gs], scales32 fp32
    [padded/gs]) with gs coerced as the reference coerces it."""
    gs = e8r_effective_gs(group_size)
    if gs > 4096:
        raise ValueError("oracle group size limit is 4096")
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    p = padded(w.size, gs)
    codes = np.empty(p // 8, dtype=np.uint8)
    scales = np.empty(p // gs, dtype=np.uint16)
    scales32 = np.empty(p // gs, dtype=np.float32)
    lib().ojo_e8r_encode(_ptr(w), w.size, gs, _ptr(codes), _ptr(scales), _ptr(scales32),
                         int(nthreads))
    return codes, scales, scales32


def e8r_decode(codes: np.ndarray, scales: np.ndarray, numel: int, group_size: int,
               dtype: int = DT_F32) -> np.ndarray:
    """RootE8LatticePacker.unpack: fp32 values, or fp16 / bf16 bit patterns."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    out = np.empty(numel, dtype=np.float32 if dtype == DT_F32 else np.uint16)
    lib().ojo_e8r_decode(_ptr(codes), _ptr(scales), numel, int(group_size), int(dtype),
                         _ptr(out))
    return out


def e8r_gemm_f64(x: np.ndarray, codes: np.ndarray, scales: np.ndarray,
                 bias: Optional[np.ndarray], N: int, K: int, group_size: int,
                 w_dtype: int = DT_F32) -> np.ndarray:
    """fp64-accumulated x @ Wdeq^T + bias, Wdeq by the 1-bit dtype rule."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    M = x.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().ojo_e8r_gemm_f64(_ptr(x), _ptr(np.ascontiguousarray(codes)),
                           _ptr(np.ascontiguousarray(scales, dtype=np.uint16)),
                           None if b is None else _ptr(b), _ptr(y), M, N, K,
                           int(group_size), int(w_dtype))
    return y


def e8r_gemm_bwd_f64(gy: np.ndarray, codes: np.ndarray, scales: np.ndarray, N: int, K: int,
                     group_size: int, w_dtype: int = DT_F32) -> np.ndarray:
    gy = np.ascontiguousarray(gy, dtype=np.float32).reshape(-1, N)
    M = gy.shape[0]
    gx = np.empty((M, K), dtype=np.float64)
    lib().ojo_e8r_gemm_bwd_f64(_ptr(gy), _ptr(np.ascontiguousarray(codes)),
                               _ptr(np.ascontiguousarray(scales, dtype=np.uint16)), _ptr(gx),
                               M, N, K, int(group_size), int(w_dtype))
    return gx


# --------------------------------------------------------------------------- Conway-Sloane / STE

def cs_project(x: np.ndarray) -> np.ndarray:
    """conway_sloane_e8_project's torch path (lattice.py:180-203) over [..., 8], fp32 or fp64."""
    if x.dtype == np.float64:
        a = np.ascontiguousarray(x)
        out = np.empty_like(a)
        lib().ojo_e8_cs_project_f64(_ptr(a), _ptr(out), a.size // 8)
    else:
        a = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(a)
        lib().ojo_e8_cs_project_f32(_ptr(a), _ptr(out), a.size // 8)
    return out


def ste_quantize(w: np.ndarray) -> np.ndarray:
    """_E8STEFunction.forward (lattice.py:853-865) on fp32 weights."""
    a = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(a)
    lib().ojo_e8_ste_quantize_f32(_ptr(a), a.size, _ptr(out))
    return out


def cs_project_half(x: np.ndarray, bf16: bool) -> np.ndarray:
    """The projection on an fp16 (bf16=False) or bf16 tensor, every op rounded to the type;
    ``x`` holds the tensor's values as fp32 (exact), the result likewise."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(a)
    lib().ojo_e8_cs_project_half(_ptr(a), _ptr(out), a.size // 8, int(bf16))
    return out


def ste_quantize_half(w: np.ndarray, bf16: bool) -> np.ndarray:
    """_E8STEFunction.forward on fp16 (bf16=False) or bf16 weights held as fp32 values."""
    a = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(a)
    lib().ojo_e8_ste_quantize_half(_ptr(a), a.size, _ptr(out), int(bf16))
    return out
