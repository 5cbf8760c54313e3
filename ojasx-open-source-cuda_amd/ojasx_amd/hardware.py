"""The ``ojasx3.hardware`` entry for the E8 path on gfx950 (MI355X).

Drop-in names for ojasx3/hardware/__init__.py, which re-exports
ojasx2/tilelang_kernels.py:

* ``TileConfig`` (tilelang_kernels.py:75-90) and
  ``TileLangHardwareAutoTuner.select_tile_config`` (:93-177).  The decision table
  is the reference's ROCm row (128 x 128 x 32, panel 8, when M, N >= 128 and the
  element is at most 2 bytes or M, N >= 256; else 64 x 64 x 32, panel 4), so a
  caller that sizes buffers or reports by it sees the same tiles.  It is advisory:
  the HIP kernels pick their own launch shapes (the decode GEMV's 16-row tiles for
  M <= 16, the MFMA GEMM's 256 x 256 or 128 x 128 x 64 tiles above).
* ``dispatch_tilelang_e8_gemm`` (:370-419): the fused packed-weight linear.  The
  reference tries a TileLang JIT kernel and returns None when it is absent or the
  shape is not a multiple of 64; here every shape on a HIP device runs the
  library's kernels (bias fused), and only a tensor off the HIP device returns
  None.  ``lut_coords`` is accepted and ignored: the codebooks live in the
  kernels' constant memory.
* ``UniversalCompiledKernel`` (:426-549) and ``compile_or_emit_universal_kernel``
  (:552-615): packed uint8 weights go to the dispatcher; dense weights run
  ``F.linear`` (and ``relu2_ballot`` the ReLU^2 + 32-column sign-mask form,
  tile_fallback.py:25-52).  There is no runtime code generation: ``source`` is a
  text record of the plan (target, tiles, format, the C entry points used).

Only ROCm targets are accepted ("auto", "cuda" -- torch's name for the HIP device
-- "rocm", "hip", "amd", "cdna", "gfx950", ...); other architectures raise
``RuntimeError`` as the reference's ``normalize_device`` does for unknown ones.
"""

from __future__ import annotations

from typing import Any, Callable, Dict, NamedTuple, Optional, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .lattice import _get_packer_for_bitrate

__all__ = [
    "TileConfig",
    "TileLangHardwareAutoTuner",
    "UniversalCompiledKernel",
    "compile_or_emit_universal_kernel",
    "dispatch_tilelang_e8_gemm",
    "is_tilelang_available",
    "normalize_target_arch",
]

_ROCM_ALIASES = {"auto", "cuda", "rocm", "hip", "amd", "cdna", "cdna3", "cdna4", "gfx90a",
                 "gfx942", "gfx950", "mi300", "mi300x", "mi355", "mi355x"}


class TileConfig(NamedTuple):
    """``(block_m, block_n, block_k, panel_size, target_arch)`` (tilelang_kernels.py:75-90)."""

    block_m: int
    block_n: int
    block_k: int
    panel_size: int
    target_arch: str

    def to_dict(self) -> Dict[str, Any]:
        return {"block_m": self.block_m, "block_n": self.block_n, "block_k": self.block_k,
                "panel_size": self.panel_size, "target_arch": self.target_arch}


def normalize_target_arch(target_arch: Union[str, torch.device, None]) -> str:
    """Canonical target of a device or alias (tile_fallback.py:588-620, ROCm rows).

    Returns "rocm" for every alias of the HIP device; raises ``RuntimeError`` for
    the reference's other targets (metal, sycl, ascend, cpu, ...), which this
    library does not run on."""
    if target_arch is None:
        raw = "auto"
    elif isinstance(target_arch, torch.device):
        raw = target_arch.type
    else:
        raw = str(target_arch).strip().lower()
    if ":" in raw:
        raw = raw.split(":", 1)[0]
    if raw in _ROCM_ALIASES:
        return "rocm"
    raise RuntimeError(
        f"Unsupported target_arch: {target_arch!r} (this library runs on gfx950 / ROCm only)")


def is_tilelang_available() -> bool:
    """tilelang_kernels.py:180: TileLang is not used; the HIP kernels are always the backend."""
    return False


class TileLangHardwareAutoTuner:
    """Tile choice of the reference's ROCm row (tilelang_kernels.py:93-177)."""

    SUPPORTED_ARCHITECTURES = ("rocm",)

    @classmethod
    def normalize_device(cls, device: Union[str, torch.device, None] = "auto") -> str:
        return normalize_target_arch(device)

    @classmethod
    def _dtype_bytes(cls, dtype: Union[torch.dtype, str, None]) -> int:
        """Element size as tilelang_kernels.py:121-141 reads it (strings by their digits)."""
        if dtype is None:
            return 2
        if isinstance(dtype, torch.dtype):
            if dtype in (torch.float16, torch.bfloat16):
                return 2
            if dtype in (torch.int8, torch.uint8):
                return 1
            return 8 if dtype == torch.float64 else 4
        s = str(dtype).lower()
        for digits, size in (("16", 2), ("8", 1), ("64", 8)):
            if digits in s:
                return size
        return 4

    @classmethod
    def select_tile_config(cls, M: int, N: int, K: int,
                           device: Union[str, torch.device, None] = "auto",
                           dtype: Union[torch.dtype, str, None] = torch.float16) -> TileConfig:
        if M <= 0 or N <= 0 or K <= 0:
            raise ValueError(f"Matrix dimensions (M, N, K) must be positive, got ({M}, {N}, {K})")
        arch = cls.normalize_device(device)
        wide = cls._dtype_bytes(dtype) <= 2 or (M >= 256 and N >= 256)
        if M >= 128 and N >= 128 and wide:
            return TileConfig(128, 128, 32, 8, arch)
        return TileConfig(64, 64, 32, 4, arch)


_LINEAR_BY_BITRATE = {1.5: ops.e8t_linear, 1.0: ops.e8r_linear}
_ENTRY_BY_BITRATE = {1.5: "ojx_e8t_gemm_fwd", 1.0: "ojx_e8r_gemm_fwd"}


def dispatch_tilelang_e8_gemm(x_2d: torch.Tensor, packed_weight: torch.Tensor,
                              block_scales: torch.Tensor, bias: Optional[torch.Tensor],
                              out_features: int, in_features: int, group_size: int,
                              bitrate: float,
                              lut_coords: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """``y[M, out] = x_2d . W^T (+ bias)`` on the HIP kernels (tilelang_kernels.py:370-419).

    Returns None only when ``x_2d`` is not on the HIP device (the reference's
    "not eligible" answer).  Layout errors raise ``RuntimeError`` from the ops
    instead of being swallowed, so a bad buffer is never silently re-routed."""
    if x_2d.device.type != "cuda":
        return None
    linear = _LINEAR_BY_BITRATE.get(float(bitrate), ops.e8_linear)
    return linear(x_2d, packed_weight.to(x_2d.device), block_scales.to(x_2d.device),
                  None if bias is None else bias.to(x_2d.device), int(out_features),
                  int(in_features), int(group_size))


def _relu2_ballot(x: torch.Tensor, weight: torch.Tensor,
                  bias: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """ReLU^2 of a dense linear and its sign mask, bit j of word w set when column
    32 w + j is positive (tile_fallback.py:25-36, 50-52)."""
    z = F.linear(x, weight, bias)
    cols = z.shape[-1]
    words = (cols + 31) // 32
    if z.numel() == 0:
        return F.relu(z).square(), z.new_empty((*z.shape[:-1], words), dtype=torch.int32)
    bits = F.pad((z.contiguous() > 0).to(torch.int64), (0, words * 32 - cols))
    shifts = torch.arange(32, device=z.device, dtype=torch.int64)
    mask = (bits.reshape(*z.shape[:-1], words, 32) << shifts).sum(-1).to(torch.int32)
    return F.relu(z).square(), mask


class UniversalCompiledKernel:
    """Callable dispatcher of one (M, N, K) problem (tilelang_kernels.py:426-549)."""

    def __init__(self, M: int, N: int, K: int, tile_config: TileConfig, source: str,
                 bitrate: float = 2.0, group_size: int = 32,
                 jit_kernel: Optional[Callable[..., Any]] = None) -> None:
        self.M, self.N, self.K = int(M), int(N), int(K)
        self.tile_config = tile_config
        self.block_m = tile_config.block_m
        self.block_n = tile_config.block_n
        self.block_k = tile_config.block_k
        self.panel_size = tile_config.panel_size
        self.target_arch = tile_config.target_arch
        self.source = source
        self.bitrate = float(bitrate)
        self.group_size = int(group_size)
        self.jit_kernel = jit_kernel
        self.backend = "hip_gfx950"

    def to_dict(self) -> Dict[str, Any]:
        return {"M": self.M, "N": self.N, "K": self.K, "block_m": self.block_m,
                "block_n": self.block_n, "block_k": self.block_k,
                "panel_size": self.panel_size, "target_arch": self.target_arch,
                "tile_config": self.tile_config, "source": self.source,
                "bitrate": self.bitrate, "group_size": self.group_size,
                "backend": self.backend, "callable": self}

    def __getitem__(self, key: str) -> Any:
        return self.to_dict()[key]

    def __contains__(self, item: str) -> bool:
        return item in self.to_dict() or (isinstance(item, str) and item in self.source)

    def __str__(self) -> str:
        return self.source

    def forward_relu2_ballot(self, x: torch.Tensor, weight: torch.Tensor,
                             bias: Optional[torch.Tensor] = None
                             ) -> Tuple[torch.Tensor, torch.Tensor]:
        w = weight.to(device=x.device, dtype=x.dtype)
        b = bias.to(device=x.device, dtype=x.dtype) if bias is not None else None
        return _relu2_ballot(x, w, b)

    def __call__(self, x: torch.Tensor, weight_or_layer: Union[torch.Tensor, nn.Module],
                 scales_or_bias: Optional[torch.Tensor] = None,
                 bias: Optional[torch.Tensor] = None,
                 lut_coords: Optional[torch.Tensor] = None, *, relu2_ballot: bool = False
                 ) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
        if isinstance(weight_or_layer, nn.Module):
            if hasattr(weight_or_layer, "forward_fused"):
                return weight_or_layer.forward_fused(x)
            return weight_or_layer(x)
        weight = weight_or_layer
        if weight.dtype == torch.uint8:
            if scales_or_bias is None:
                raise ValueError(
                    "block_scales must be provided when calling with uint8 packed_weight")
            if x.device.type != "cuda":
                raise RuntimeError(
                    "packed E8 weights run on the HIP device; move x to 'cuda' first")
            _get_packer_for_bitrate(self.bitrate)
            in_features = x.shape[-1]
            x_2d = x.reshape(-1, in_features).contiguous()
            y = dispatch_tilelang_e8_gemm(x_2d, weight, scales_or_bias, bias, self.N,
                                          in_features, self.group_size, self.bitrate,
                                          lut_coords)
            return y.reshape(*x.shape[:-1], self.N)
        dense_bias = scales_or_bias if bias is None else bias
        w = weight.to(device=x.device, dtype=x.dtype)
        b = dense_bias.to(device=x.device, dtype=x.dtype) if dense_bias is not None else None
        if relu2_ballot:
            return _relu2_ballot(x, w, b)
        return F.linear(x, w, b)


def _plan_source(M: int, N: int, K: int, cfg: TileConfig, bitrate: float,
                 group_size: int, dtype: Union[torch.dtype, str, None]) -> str:
    entry = _ENTRY_BY_BITRATE.get(float(bitrate), "ojx_e8_gemm_fwd")
    fmt = {1.5: "ternary E8, 3 bytes per 16 weights", 1.0: "Root E8, 1 byte per 8 weights"
           }.get(float(bitrate), "2-bit E8, 1 byte per 4 weights")
    regime = ("decode GEMV (weights streamed once, codes expanded in registers)" if M <= 16
              else "MFMA GEMM (LDS-staged tiles, K split for small grids)")
    return "\n".join([
        f"// ojasx_amd E8 linear plan for gfx950 (MI355X): y[{M}, {N}] = x[{M}, {K}] . W^T",
        f"// weights: {fmt}, group_size {group_size}, fp16 block scales",
        f"// compute dtype: {dtype}; accumulation fp32",
        f"// kernel: {regime}",
        f"// C entry point: {entry} (libojasx_e8t.so)",
        f"// tile_config: block_m={cfg.block_m} block_n={cfg.block_n} block_k={cfg.block_k} "
        f"panel_size={cfg.panel_size} target_arch={cfg.target_arch}",
    ])


def compile_or_emit_universal_kernel(M: int, N: int, K: int,
                                     device: Union[str, torch.device, None] = "auto",
                                     bitrate: float = 2.0, group_size: int = 32,
                                     dtype: Union[torch.dtype, str, None] = torch.float16
                                     ) -> UniversalCompiledKernel:
    """tilelang_kernels.py:552-615 without code generation: the kernels are prebuilt."""
    cfg = TileLangHardwareAutoTuner.select_tile_config(M, N, K, device=device, dtype=dtype)
    return UniversalCompiledKernel(M=M, N=N, K=K, tile_config=cfg,
                                   source=_plan_source(M, N, K, cfg, bitrate, group_size, dtype),
                                   bitrate=bitrate, group_size=group_size)
