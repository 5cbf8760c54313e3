"""Torch-op restatement of the reference's portable CPU forward -- TEST/BENCH ONLY.

This is the CPU baseline that ``bench.py`` times beside the GPU (kind "port"):
the path a Linux user of the reference gets, because the reference's native
math extension is only built on Darwin (``setup.py:104-110``), so
``_FusedE8GEMMFunction.forward`` falls through to
``unpack(use_workspace=True)`` + ``F.linear`` (``ojasx2/math/lattice.py:610-624``).

Steps restated (no reference code is imported or copied):
  * codebook   lattice.py:309-318 -- rank r <-> raw 2r, digits of raw in base 3
  * unpack     lattice.py:393-419 -- bytes -> two 12-bit codes, LUT gather,
                                     copy into a reused workspace, multiply by
                                     the per-group scale cast to the x dtype
  * forward    lattice.py:613-624 -- F.linear(x, W, bias)
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

_LUT: Optional[torch.Tensor] = None
_WS: dict = {}


def rank_to_coords() -> torch.Tensor:
    global _LUT
    if _LUT is None:
        raw = torch.arange(3281, dtype=torch.int64) * 2
        digits = []
        for _ in range(8):
            digits.append(raw % 3 - 1)
            raw = raw // 3
        _LUT = torch.stack(digits, dim=1).to(torch.int8)
    return _LUT


def unpack(packed: torch.Tensor, scales: torch.Tensor, shape, dtype=torch.float32,
           use_workspace: bool = True) -> torch.Tensor:
    lut = rank_to_coords()
    trip = packed.view(-1, 3)
    b0 = trip[:, 0].to(torch.int32)
    b1 = trip[:, 1].to(torch.int32)
    b2 = trip[:, 2].to(torch.int32)
    codes = torch.empty((trip.shape[0], 2), dtype=torch.int32)
    codes[:, 0] = b0 | ((b1 & 0x0F) << 8)
    codes[:, 1] = ((b1 >> 4) & 0x0F) | (b2 << 4)
    total = shape[0] * shape[1]
    padded = trip.shape[0] * 16
    gs = padded // max(1, scales.numel())
    coords = lut[codes.view(-1)].view(-1, gs)
    if use_workspace and padded == total:
        key = dtype
        buf = _WS.get(key)
        if buf is None or buf.numel() < total:
            buf = torch.empty(total, dtype=dtype)
            _WS[key] = buf
        out = buf[:total].view(-1, gs)
        out.copy_(coords)
        out.mul_(scales.to(dtype).view(-1, 1))
        return out.view(shape)
    full = (coords.to(dtype) * scales.to(dtype).view(-1, 1)).reshape(-1)
    return full[:total].view(shape)


def linear(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor,
           bias: Optional[torch.Tensor], out_features: int, in_features: int) -> torch.Tensor:
    x2 = x.reshape(-1, in_features)
    w = unpack(packed, scales, (out_features, in_features), dtype=x2.dtype, use_workspace=True)
    b = bias.to(x2.dtype) if bias is not None else None
    return F.linear(x2, w, b).reshape(*x.shape[:-1], out_features)
