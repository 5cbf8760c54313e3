"""E8 lattice quantization (ternary 1.5, 2 and 1 bit/weight) on MI355X.

Mirrors the E8 parts of ``ojasx3.lattice`` / ``ojasx2.math.lattice``
-- same names, arguments, buffers, coercions and errors -- with every array
operation on the path running in the HIP kernels behind ``ojasx_amd.ops``:

=================================  ==========================================
this module                         reference (ojasx2/math/lattice.py)
=================================  ==========================================
``fwht_block32``                    :91-102
``fast_walsh_hadamard_transform``   :104-122
``randomized_hadamard_transform``   :125-155
``conway_sloane_e8_project``        :162-203   -> ops.cs_project
``_E8STEFunction``                  :853-869   -> ops.ste_quantize
``E8QuantizationAwareLinear``       :872-898
``_get_ternary_e8_luts``            :292-332
``TernaryE8LatticePacker.pack``     :338-384   -> ops.encode (one HIP kernel)
``TernaryE8LatticePacker.unpack``   :386-419   -> ops.decode
``E8LatticePacker.pack``            :213-249   -> ops.encode2 (2-bit)
``E8LatticePacker.unpack``          :252-279   -> ops.decode2
``_get_root_e8_lut``                :428-466
``RootE8LatticePacker.pack``        :473-509   -> ops.encode1 (1-bit)
``RootE8LatticePacker.unpack``      :512-533   -> ops.decode1
``_get_packer_for_bitrate``         :536-541
``_FusedE8GEMMFunction``            :548-717   -> ops.e8t_linear / ops.e8_linear
``E8LatticeLinear``                 :724-846
``pack_model_e8``                   :901-945
=================================  ==========================================

Bitrates 1.5 (ternary), 2.0 (2-bit, the reference's default for any bitrate other
than 1.0 and 1.5) and 1.0 (RootE8LatticePacker) are implemented.
CPU tensors given to ``pack`` / ``unpack`` are processed on the current GPU and
the result is returned on the CPU; the fused forward requires GPU tensors.
"""

from __future__ import annotations

import copy
import math
from typing import Dict, Optional, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops

__all__ = [
    "fwht_block32",
    "fast_walsh_hadamard_transform",
    "randomized_hadamard_transform",
    "TernaryE8LatticePacker",
    "E8LatticePacker",
    "RootE8LatticePacker",
    "_FusedE8GEMMFunction",
    "conway_sloane_e8_project",
    "_E8STEFunction",
    "E8QuantizationAwareLinear",
    "E8LatticeLinear",
    "pack_model_e8",
]

_HADAMARD_NORM = 0.1767766952966369  # 1/sqrt(32), as a python float (lattice.py:101)


def fwht_block32(x: torch.Tensor) -> torch.Tensor:
    """Normalised 32-point Walsh-Hadamard transform along the last dim (lattice.py:91-102).

    Radix-2 butterflies at distances 1, 2, 4, 8, 16 (sum to the lower index,
    difference to the upper), then one multiply by 1/sqrt(32): the same sequence
    of rounded operations as the reference, so packed codes of a Hadamard layer
    match bit for bit.  GPU tensors (fp32/fp16/bf16/fp64) run one HIP kernel
    (``ops.fwht32``, differentiable); tensors on the CPU are transformed there
    with torch stages, as the reference transforms them.  Returns ``x``
    unchanged if the last dim is not a positive multiple of 32."""
    shape = x.shape
    if shape[-1] == 0 or shape[-1] % 32 != 0:
        return x
    if x.is_cuda and x.dtype in ops._FWHT_CODE:
        return ops.fwht32(x)  # one HIP kernel, the same rounded operations
    h = x.reshape(-1, 32)
    for dist in (1, 2, 4, 8, 16):
        v = h.reshape(-1, 32 // (2 * dist), 2, dist)
        a, b = v[:, :, 0, :], v[:, :, 1, :]
        h = torch.stack([a + b, a - b], dim=2).reshape(-1, 32)
    return (h * _HADAMARD_NORM).reshape(shape)


def conway_sloane_e8_project(x: torch.Tensor, prefer_native: bool = True) -> torch.Tensor:
    """Snaps every 8-vector of x to the nearest point of E8 = D8 U (D8 + 1/2) (lattice.py:162-203).

    One HIP kernel, with the arithmetic of the reference's torch path (round half to even;
    an odd sum moves the first coordinate with the largest rounding error towards x; D8
    wins ties of the squared distances).  ``prefer_native`` selected the reference's CPU
    kernel, which rounds halves away from zero; it is accepted and ignored.  fp32, fp64, and
    fp16 / bf16 tensors (every op rounded to the dtype, as the reference's torch expressions
    compute on such a tensor); CPU tensors are processed on the current GPU and returned on
    the CPU."""
    del prefer_native
    if x.shape[-1] != 8:
        raise ValueError(f"Last dimension must be 8 for E8 lattice (got {x.shape[-1]}).")
    if x.numel() == 0:
        return x.clone()
    out = ops.cs_project(_on_gpu(x))
    return out.to(x.device) if x.device.type != "cuda" else out


class _E8STEFunction(torch.autograd.Function):
    """Straight-through E8 weight quantizer (lattice.py:853-869): the forward snaps each flat
    8-vector, scaled by its norm / sqrt(8) + 1e-8, to E8 (one HIP kernel, in the weight's
    dtype: fp32, or fp16 / bf16 with every op rounded to it as in the reference); the
    backward passes the gradient through unchanged."""

    @staticmethod
    def forward(ctx, w: torch.Tensor) -> torch.Tensor:
        out = ops.ste_quantize(_on_gpu(w))
        return out.to(w.device) if w.device.type != "cuda" else out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor) -> torch.Tensor:
        return grad_output


class E8QuantizationAwareLinear(nn.Module):
    """nn.Linear whose weight passes through the E8 straight-through quantizer in every
    forward (lattice.py:872-898)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 device: Optional[torch.device] = None, dtype: Optional[torch.dtype] = None
                 ) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.empty(out_features, in_features, device=device,
                                               dtype=dtype))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, device=device, dtype=dtype))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            fan_in, _ = nn.init._calculate_fan_in_and_fan_out(self.weight)
            bound = 1 / math.sqrt(fan_in) if fan_in > 0 else 0
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w_q = _E8STEFunction.apply(self.weight)
        return F.linear(x, w_q, self.bias)


def fast_walsh_hadamard_transform(x: torch.Tensor) -> torch.Tensor:
    """Normalised Walsh-Hadamard transform along a power-of-two last dim (lattice.py:104-122).

    fwht_block32 for n = 32; otherwise butterflies at distances 1, 2, 4, ... (sum to the
    lower index, difference to the upper) and one true division by sqrt(n): the reference's
    sequence of rounded operations, on the tensor's own device."""
    n = x.shape[-1]
    if n <= 0 or (n & (n - 1)) != 0:
        raise ValueError(f"Last dimension ({n}) must be a positive power of 2 for FWHT.")
    if n == 32:
        return fwht_block32(x)
    h, d = x.reshape(-1, n), 1
    while d < n:
        v = h.reshape(-1, n // (2 * d), 2, d)
        h = torch.stack([v[:, :, 0, :] + v[:, :, 1, :], v[:, :, 0, :] - v[:, :, 1, :]], dim=2)
        d *= 2
    return h.reshape(x.shape) / math.sqrt(n)


def randomized_hadamard_transform(w: torch.Tensor, seed: Optional[int] = 42
                                  ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Randomised Hadamard rotation of a weight matrix (lattice.py:125-155): random row and
    column signs s1, s2 drawn from a generator on w's device seeded with ``seed`` (the same
    draws as the reference on the same device), then the two-sided transform when both
    dims are powers of two, else fwht_block32 along rows of a multiple-of-32 width.
    Returns (w_rot, s1, s2)."""
    m, n = w.shape
    rng = torch.Generator(device=w.device)
    if seed is not None:
        rng.manual_seed(seed)
    s1 = torch.randint(0, 2, (m,), generator=rng, device=w.device, dtype=w.dtype) * 2 - 1
    s2 = torch.randint(0, 2, (n,), generator=rng, device=w.device, dtype=w.dtype) * 2 - 1
    signed = (w * s2.unsqueeze(0)) * s1.unsqueeze(1)
    if m & (m - 1) == 0 and n & (n - 1) == 0:
        rot = fast_walsh_hadamard_transform(signed)
        rot = fast_walsh_hadamard_transform(rot.transpose(0, 1)).transpose(0, 1)
    elif n % 32 == 0:
        rot = fwht_block32(signed)
    else:
        rot = signed
    return rot, s1, s2


_DEVICE_TERNARY_LUTS: Dict[Tuple[str, Optional[int]], Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = {}


def _get_ternary_e8_luts(device: Optional[torch.device] = None
                         ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(rank_to_coords int8 [3281, 8], raw_to_rank int64 [6561], powers int64 [8]).

    Same tables as lattice.py:292-332, built from the closed form raw = 2 * rank
    (the enumeration keeps even digit sums, and 3^i is odd).  The HIP kernels do
    not use them; they are provided for callers of the reference API."""
    if device is None:
        key = ("cpu", None)
    else:
        device = torch.device(device)
        key = (device.type, device.index)
    if key not in _DEVICE_TERNARY_LUTS:
        raw = torch.arange(3281, dtype=torch.int64) * 2
        digits = []
        r = raw.clone()
        for _ in range(8):
            digits.append(r % 3 - 1)
            r = r // 3
        rank_to_coords = torch.stack(digits, dim=1).to(torch.int8)
        raw_to_rank = torch.zeros(6561, dtype=torch.int64)
        raw_to_rank[raw] = torch.arange(3281, dtype=torch.int64)
        powers = torch.tensor([3 ** i for i in range(8)], dtype=torch.int64)
        dev = torch.device(key[0], key[1]) if key[1] is not None else torch.device(key[0])
        _DEVICE_TERNARY_LUTS[key] = (rank_to_coords.to(dev), raw_to_rank.to(dev), powers.to(dev))
    return _DEVICE_TERNARY_LUTS[key]


def _on_gpu(t: torch.Tensor) -> torch.Tensor:
    if t.device.type == "cuda":
        return t
    if not torch.cuda.is_available():
        raise RuntimeError("ojasx_amd needs a ROCm GPU; no device is available")
    return t.to("cuda")


class TernaryE8LatticePacker:
    """Packs weight matrices into 1.50 bits/weight using D8 cap {-1, 0, +1}^8 (3,281 points)."""

    @staticmethod
    def pack(w: torch.Tensor, group_size: int = 32
             ) -> Tuple[torch.Tensor, torch.Tensor, Tuple[int, int]]:
        m, n = w.shape
        if group_size <= 0 or group_size % 16 != 0:
            group_size = 16  # silent coercion, lattice.py:346-347
        packed, scales = ops.encode(_on_gpu(w), group_size)
        if w.device.type != "cuda":
            packed, scales = packed.to(w.device), scales.to(w.device)
        return packed, scales, (m, n)

    @staticmethod
    def unpack(packed_codes: torch.Tensor, scales: torch.Tensor, shape: Tuple[int, int],
               dtype: torch.dtype = torch.float32, use_workspace: bool = False) -> torch.Tensor:
        # use_workspace selected a shared scratch buffer in the reference
        # (lattice.py:62-84); here every call returns a fresh tensor.
        del use_workspace
        total = shape[0] * shape[1]
        padded = (packed_codes.numel() // 3) * 16
        group_size = padded // max(1, scales.numel())  # inferred as in lattice.py:407-409
        out = ops.decode(_on_gpu(packed_codes), _on_gpu(scales).to(torch.float16), total,
                         group_size, dtype)
        if packed_codes.device.type != "cuda":
            out = out.to(packed_codes.device)
        return out.view(shape)


class E8LatticePacker:
    """Packs weight matrices into 2.0 bits/weight (4 weights per uint8 byte) with auto-padding."""

    @staticmethod
    def pack(w: torch.Tensor, group_size: int = 8
             ) -> Tuple[torch.Tensor, torch.Tensor, Tuple[int, int]]:
        m, n = w.shape
        if group_size <= 0 or group_size % 8 != 0:
            raise ValueError(f"group_size ({group_size}) must be a positive multiple of 8.")
        packed, scales = ops.encode2(_on_gpu(w), group_size)
        if w.device.type != "cuda":
            packed, scales = packed.to(w.device), scales.to(w.device)
        return packed, scales, (m, n)

    @staticmethod
    def unpack(packed_codes: torch.Tensor, scales: torch.Tensor, shape: Tuple[int, int],
               dtype: torch.dtype = torch.float32, use_workspace: bool = False) -> torch.Tensor:
        del use_workspace  # a shared scratch buffer in the reference; a fresh tensor here
        total = shape[0] * shape[1]
        padded = packed_codes.numel() * 4
        group_size = padded // max(1, scales.numel())  # inferred as in lattice.py:264-266
        out = ops.decode2(_on_gpu(packed_codes), _on_gpu(scales).to(torch.float16), total,
                          group_size, dtype)
        if packed_codes.device.type != "cuda":
            out = out.to(packed_codes.device)
        return out.view(shape)


_DEVICE_ROOT_E8_LUTS: Dict[Tuple[str, Optional[int]], torch.Tensor] = {}


def _get_root_e8_lut(device: Optional[torch.device] = None) -> torch.Tensor:
    """The 256 x 8 fp32 table of lattice.py:428-466 (scaled by 2): the 112 rows with +-2 at
    two coordinates, the 128 rows (+-1)^8 with an even number of -1 (itertools.product
    order), the 16 rows with +-2 at one coordinate.  The HIP kernels carry the same table
    (csrc/e8t_root.h); this copy is for callers of the reference API."""
    if device is None:
        key = ("cpu", None)
    else:
        device = torch.device(device)
        key = (device.type, device.index)
    if key not in _DEVICE_ROOT_E8_LUTS:
        rows = []
        for i in range(8):
            for j in range(i + 1, 8):
                for s1 in (-1.0, 1.0):
                    for s2 in (-1.0, 1.0):
                        r = [0.0] * 8
                        r[i], r[j] = s1, s2
                        rows.append(r)
        for p in range(256):
            signs = [0.5 if (p >> (7 - k)) & 1 else -0.5 for k in range(8)]
            if sum(1 for v in signs if v < 0) % 2 == 0:
                rows.append(signs)
        for i in range(8):
            for s in (-1.0, 1.0):
                r = [0.0] * 8
                r[i] = s
                rows.append(r)
        lut = torch.tensor(rows, dtype=torch.float32) * 2.0
        dev = torch.device(key[0], key[1]) if key[1] is not None else torch.device(key[0])
        _DEVICE_ROOT_E8_LUTS[key] = lut.to(dev)
    return _DEVICE_ROOT_E8_LUTS[key]


class RootE8LatticePacker:
    """Packs weight matrices into 1.00 bit/weight (1 byte per 8D vector) using the 240 E8 roots."""

    @staticmethod
    def pack(w: torch.Tensor, group_size: int = 32
             ) -> Tuple[torch.Tensor, torch.Tensor, Tuple[int, int]]:
        m, n = w.shape
        if group_size <= 0 or group_size % 8 != 0:
            group_size = 8  # silent coercion, lattice.py:485-486
        codes, scales = ops.encode1(_on_gpu(w), group_size)
        if w.device.type != "cuda":
            codes, scales = codes.to(w.device), scales.to(w.device)
        return codes, scales, (m, n)

    @staticmethod
    def unpack(packed_codes: torch.Tensor, scales: torch.Tensor, shape: Tuple[int, int],
               dtype: torch.dtype = torch.float32, use_workspace: bool = False) -> torch.Tensor:
        del use_workspace  # a shared scratch buffer in the reference; a fresh tensor here
        total = shape[0] * shape[1]
        padded = packed_codes.numel() * 8
        group_size = padded // max(1, scales.numel())  # inferred as in lattice.py:524-525
        out = ops.decode1(_on_gpu(packed_codes), _on_gpu(scales).to(torch.float16), total,
                          group_size, dtype)
        if packed_codes.device.type != "cuda":
            out = out.to(packed_codes.device)
        return out.view(shape)


def _get_packer_for_bitrate(bitrate: float):
    """lattice.py:536-541: 1.0 -> RootE8LatticePacker, 1.5 -> TernaryE8LatticePacker,
    anything else -> E8LatticePacker."""
    if bitrate == 1.0:
        return RootE8LatticePacker
    if bitrate == 1.5:
        return TernaryE8LatticePacker
    return E8LatticePacker


def _require_supported(bitrate: float) -> None:
    _get_packer_for_bitrate(float(bitrate))


class _FusedE8GEMMFunction(torch.autograd.Function):
    """Fused decode-in-register E8 linear (lattice.py:548-717), one HIP route.

    Same ``apply`` arguments as the reference: (x, packed_weight, block_scales,
    bias, out_features, in_features, group_size, bitrate, use_hadamard).  Saves
    only the packed buffers for backward; returns grads for x and bias."""

    MAX_EPHEMERAL_ELEMENTS: int = 67_108_864  # kept for API parity; no workspace is used

    @staticmethod
    def forward(ctx, x, packed_weight, block_scales, bias, out_features, in_features,
                group_size, bitrate, use_hadamard=False):
        _require_supported(bitrate)
        x_rot = fwht_block32(x) if (use_hadamard and in_features % 32 == 0) else x
        ctx.save_for_backward(packed_weight, block_scales)
        ctx.dims = (out_features, in_features, group_size)
        ctx.bitrate = float(bitrate)
        ctx.x_shape = x_rot.shape
        ctx.has_bias = bias is not None
        ctx.use_hadamard = use_hadamard
        linear = {1.5: ops.e8t_linear, 1.0: ops.e8r_linear}.get(ctx.bitrate, ops.e8_linear)
        return linear(x_rot, packed_weight, block_scales, bias, out_features, in_features,
                      group_size)

    @staticmethod
    def backward(ctx, grad_y):
        packed_weight, block_scales = ctx.saved_tensors
        out_features, in_features, group_size = ctx.dims
        bwd = {1.5: ops.e8t_linear_bwd_dx, 1.0: ops.e8r_linear_bwd_dx}.get(
            ctx.bitrate, ops.e8_linear_bwd_dx)
        grad_x = bwd(grad_y.contiguous(), packed_weight, block_scales, out_features,
                     in_features, group_size)
        grad_x = grad_x.reshape(ctx.x_shape)
        if ctx.use_hadamard and in_features % 32 == 0:
            grad_x = fwht_block32(grad_x)
        grad_bias = grad_y.reshape(-1, out_features).sum(dim=0) if ctx.has_bias else None
        return grad_x, None, None, grad_bias, None, None, None, None, None


class E8LatticeLinear(nn.Module):
    """Linear layer with base weights packed into the 8D E8 lattice (lattice.py:724-846).

    Buffers ``packed_weight`` (uint8 [padded*3/16] at bitrate 1.5, [padded/4] at 2.0,
    [padded/8] at 1.0)
    and ``block_scales`` (fp16 [padded/group]) have the reference's names, shapes and
    layout, so its state_dicts load unchanged.  LoRA adapters as in the reference."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, rank: int = 0,
                 lora_alpha: float = 16.0, group_size: int = 8, bitrate: float = 2.0,
                 use_hadamard: bool = False, device: Optional[torch.device] = None,
                 dtype: Optional[torch.dtype] = None) -> None:
        super().__init__()
        _require_supported(bitrate)
        self.in_features = in_features
        self.out_features = out_features
        self.rank = rank
        self.lora_alpha = lora_alpha
        self.scaling = (lora_alpha / rank) if rank > 0 else 0.0
        self.bitrate = float(bitrate)
        self.use_hadamard = bool(use_hadamard and (in_features % 32 == 0))

        total = out_features * in_features
        if self.bitrate == 1.5:  # lattice.py:752-766
            eff_group = group_size if (group_size >= 16 and group_size % 16 == 0) else 16
            padded = total + ((-total) % eff_group)
            num_bytes = (padded * 3) // 16
        elif self.bitrate == 1.0:
            eff_group = group_size if (group_size >= 8 and group_size % 8 == 0) else 8
            padded = total + ((-total) % eff_group)
            num_bytes = padded // 8
        else:
            eff_group = group_size if (group_size >= 8 and group_size % 8 == 0) else 8
            padded = total + ((-total) % eff_group)
            num_bytes = padded // 4
        self.group_size = eff_group
        self.register_buffer("packed_weight",
                             torch.zeros(num_bytes, dtype=torch.uint8, device=device))
        self.register_buffer("block_scales",
                             torch.ones(padded // eff_group, dtype=torch.float16, device=device))
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=dtype, device=device))
        else:
            self.register_parameter("bias", None)
        if rank > 0:
            self.lora_A = nn.Parameter(torch.zeros(in_features, rank, dtype=dtype, device=device))
            self.lora_B = nn.Parameter(torch.zeros(rank, out_features, dtype=dtype, device=device))
            nn.init.kaiming_uniform_(self.lora_A, a=math.sqrt(5))
            nn.init.zeros_(self.lora_B)
        else:
            self.register_parameter("lora_A", None)
            self.register_parameter("lora_B", None)

    @classmethod
    def from_linear(cls, linear: nn.Linear, rank: int = 0, lora_alpha: float = 16.0,
                    group_size: int = 8, bitrate: float = 2.0,
                    use_hadamard: bool = False) -> "E8LatticeLinear":
        _require_supported(bitrate)
        eff_gs = max(16, group_size) if bitrate == 1.5 else group_size  # lattice.py:793
        m = cls(linear.in_features, linear.out_features, bias=(linear.bias is not None),
                rank=rank, lora_alpha=lora_alpha, group_size=eff_gs, bitrate=bitrate,
                use_hadamard=use_hadamard, device=linear.weight.device,
                dtype=linear.weight.dtype)
        with torch.no_grad():
            w = fwht_block32(linear.weight) if m.use_hadamard else linear.weight
            packer = _get_packer_for_bitrate(bitrate)
            packed, scales, _ = packer.pack(w, group_size=m.group_size)
            m.packed_weight.copy_(packed)
            m.block_scales.copy_(scales)
            if linear.bias is not None:
                m.bias.copy_(linear.bias)
        return m

    def unpack_weights(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        packer = _get_packer_for_bitrate(self.bitrate)
        w = packer.unpack(self.packed_weight, self.block_scales,
                          (self.out_features, self.in_features), dtype=dtype)
        return fwht_block32(w) if self.use_hadamard else w

    def forward_fused(self, x: torch.Tensor) -> torch.Tensor:
        has_lora = self.rank > 0 and self.lora_A is not None and self.lora_B is not None
        if (has_lora and not self.use_hadamard and self.lora_A.shape[-1] <= ops.LORA_MAX_RANK
                and x.is_cuda):
            # the adapter term scaling * ((x @ A) @ B) (lattice.py:839-842) added inside the
            # E8 kernel's epilogue; with a Hadamard rotation the E8 op sees the rotated x
            # while the adapter takes the original, so that case stays unfused below
            _require_supported(self.bitrate)
            fmt = {1.5: ops.FMT_TERNARY, 1.0: ops.FMT_ROOT}.get(float(self.bitrate), ops.FMT_E8)
            return ops.linear_lora(x, self.packed_weight, self.block_scales, self.bias,
                                   self.lora_A, self.lora_B, float(self.scaling), fmt,
                                   self.out_features, self.in_features, self.group_size)
        out = _FusedE8GEMMFunction.apply(x, self.packed_weight, self.block_scales, self.bias,
                                         self.out_features, self.in_features, self.group_size,
                                         self.bitrate, self.use_hadamard)
        if has_lora:
            lora_a = self.lora_A.to(x.dtype) if self.lora_A.dtype != x.dtype else self.lora_A
            lora_b = self.lora_B.to(x.dtype) if self.lora_B.dtype != x.dtype else self.lora_B
            out = out + self.scaling * ((x @ lora_a) @ lora_b)
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.forward_fused(x)


def pack_model_e8(model: nn.Module, rank: int = 0, lora_alpha: float = 16.0,
                  group_size: int = 32, bitrate: float = 2.0, use_hadamard: bool = False,
                  target_modules: Optional[Union[list, tuple, str]] = None,
                  exclude_modules: Optional[Union[list, tuple]] = None,
                  inplace: bool = True) -> nn.Module:
    """Recursively replaces nn.Linear modules by E8LatticeLinear (lattice.py:901-945)."""
    target = model if inplace else copy.deepcopy(model)
    if isinstance(target_modules, str):
        target_modules = [target_modules]
    for name, module in target.named_children():
        if exclude_modules is not None and any(ex in name for ex in exclude_modules):
            continue
        targeted = True if target_modules is None else any(t in name for t in target_modules)
        if isinstance(module, nn.Linear) and targeted:
            setattr(target, name, E8LatticeLinear.from_linear(
                module, rank=rank, lora_alpha=lora_alpha, group_size=group_size,
                bitrate=bitrate, use_hadamard=use_hadamard))
        else:
            pack_model_e8(module, rank=rank, lora_alpha=lora_alpha, group_size=group_size,
                          bitrate=bitrate, use_hadamard=use_hadamard,
                          target_modules=target_modules, exclude_modules=exclude_modules,
                          inplace=True)
    return target
