"""2-bit E8 compression of optimizer state (ojasx2/grad_free_optimizer.py:106-157).

The reference keeps a parameter's first moment (``exp_avg``) and its gradient
accumulation window E8-packed: the flat tensor, zero padded to a multiple of 32, is
packed as a [rows, 32] matrix with E8LatticePacker at group size 32 and stored under
``<name>_packed`` / ``<name>_scales`` / ``<name>_padded_rows`` in the parameter's state
dict.  These functions do the same with the HIP 2-bit codec (the state stays on the
tensor's device), so an optimizer built on the reference's helpers can switch to them.
"""

from __future__ import annotations

from typing import Any, Dict

import torch
import torch.nn.functional as F

from .lattice import E8LatticePacker

_GROUP = 32


def _pack_into(st: Dict[str, Any], name: str, tensor: torch.Tensor) -> None:
    flat = tensor.reshape(-1)
    pad = (-flat.numel()) % _GROUP
    if pad:
        flat = F.pad(flat, (0, pad))
    rows = flat.numel() // _GROUP
    packed, scales, _ = E8LatticePacker.pack(flat.view(rows, _GROUP), group_size=_GROUP)
    st[f"{name}_packed"] = packed
    st[f"{name}_scales"] = scales
    st[f"{name}_padded_rows"] = rows
    st.pop(name, None)


def _unpack_from(st: Dict[str, Any], name: str, target_shape: torch.Size,
                 dtype: torch.dtype) -> torch.Tensor:
    rows = st.get(f"{name}_padded_rows", target_shape.numel() // _GROUP)
    full = E8LatticePacker.unpack(st[f"{name}_packed"], st[f"{name}_scales"], (rows, _GROUP),
                                  dtype=dtype)
    return full.reshape(-1)[: target_shape.numel()].view(target_shape)


def unpack_exp_avg(st: Dict[str, Any], target_shape: torch.Size,
                   dtype: torch.dtype) -> torch.Tensor:
    """grad_free_optimizer.py:106-115: the decoded moment, or the dense one cast to dtype."""
    if "exp_avg_packed" in st:
        return _unpack_from(st, "exp_avg", target_shape, dtype)
    return st["exp_avg"].to(dtype)


def pack_exp_avg(st: Dict[str, Any], tensor: torch.Tensor, use_e8: bool,
                 storage_dtype: torch.dtype) -> None:
    """grad_free_optimizer.py:117-134: E8-pack tensors of at least 8 values when use_e8,
    else keep (or overwrite in place) a dense copy in storage_dtype."""
    if use_e8 and tensor.numel() >= 8:
        _pack_into(st, "exp_avg", tensor)
        return
    if st.get("exp_avg") is None:
        st["exp_avg"] = tensor.to(storage_dtype).clone()
    else:
        st["exp_avg"].copy_(tensor.to(storage_dtype))


def unpack_grad_accum(st: Dict[str, Any], target_shape: torch.Size,
                      dtype: torch.dtype) -> torch.Tensor:
    """grad_free_optimizer.py:136-145."""
    if "grad_accum_packed" in st:
        return _unpack_from(st, "grad_accum", target_shape, dtype)
    return st["grad_accum"].to(dtype)


def pack_grad_accum(st: Dict[str, Any], tensor: torch.Tensor) -> None:
    """grad_free_optimizer.py:147-157: always E8-packed."""
    _pack_into(st, "grad_accum", tensor)
