"""Row-block packing with the reference's layout contract (ojasx2/streaming_e8.py:80-159).

``pack_weight_rowwise`` packs ``row_block`` rows at a time and returns bytes
identical to whole-matrix packing whenever every row holds whole groups
(``in_features % group_size == 0``); layouts that would let a group cross a row
are rejected with the reference's ``ValueError`` messages.
"""

from __future__ import annotations

from typing import List, Tuple

import torch

from .lattice import _get_packer_for_bitrate, fwht_block32

_SUPPORTED_BITRATES = {1.0, 1.5, 2.0}


def _validate_row_layout(out_features: int, in_features: int, bitrate: float,
                         group_size: int) -> None:
    """streaming_e8.py:90-109."""
    if float(bitrate) not in _SUPPORTED_BITRATES:
        raise ValueError(f"Unsupported E8 bitrate {bitrate!r}; expected one of "
                         f"{sorted(_SUPPORTED_BITRATES)}")
    _get_packer_for_bitrate(float(bitrate))
    if out_features <= 0 or in_features <= 0:
        raise ValueError("Streaming E8 requires non-empty two-dimensional weights")
    if group_size <= 0 or group_size % 32 != 0:
        raise ValueError("The current E8 packers require group_size to be a positive multiple of 32")
    if in_features % group_size != 0:
        raise ValueError(
            f"in_features={in_features} is not divisible by group_size={group_size}. "
            "Checkpoint-direct row packing would cross a scale-group boundary and "
            "change the legacy layout; use a compatible group size or the explicit "
            "whole-matrix conversion path.")


def _pack_row_block(block: torch.Tensor, bitrate: float, group_size: int,
                    use_hadamard: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """streaming_e8.py:112-123: the Hadamard pair is part of the layer transform."""
    source = fwht_block32(block) if use_hadamard else block
    packer = _get_packer_for_bitrate(float(bitrate))
    packed, scales, _ = packer.pack(source, group_size=group_size)
    return packed, scales


def pack_weight_rowwise(weight: torch.Tensor, *, bitrate: float = 1.5, group_size: int = 32,
                        row_block: int = 32, use_hadamard: bool = False
                        ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Pack a materialised matrix ``row_block`` rows at a time (streaming_e8.py:126-159)."""
    if weight.ndim != 2:
        raise ValueError(f"Expected a rank-2 weight, got shape {tuple(weight.shape)}")
    if row_block <= 0:
        raise ValueError("row_block must be positive")
    out_features, in_features = map(int, weight.shape)
    _validate_row_layout(out_features, in_features, bitrate, group_size)
    packed_parts: List[torch.Tensor] = []
    scale_parts: List[torch.Tensor] = []
    for start in range(0, out_features, row_block):
        packed, scales = _pack_row_block(weight[start:start + row_block], bitrate, group_size,
                                         use_hadamard)
        packed_parts.append(packed)
        scale_parts.append(scales)
    return torch.cat(packed_parts), torch.cat(scale_parts)
