"""ojasx_amd -- MI355X-native E8 quantized-weight path: ternary 1.5 bit/weight,
2 bit/weight and 1 bit/weight (Root E8).

Drop-in for the E8 names of ``ojasx3.lattice``: the packer, the fused linear and
the layer keep the reference's signatures and buffer layout, and every array
operation runs in hand-written HIP kernels for gfx950 (libojasx_e8t.so, C ABI in
include/ojasx_e8t.h) registered as ``torch.ops.ojasx_e8t.*``.
"""

from . import grouped, hardware, ops, optim_state
from .lattice import (
    E8LatticeLinear,
    E8QuantizationAwareLinear,
    _E8STEFunction,
    conway_sloane_e8_project,
    fast_walsh_hadamard_transform,
    randomized_hadamard_transform,
    E8LatticePacker,
    RootE8LatticePacker,
    TernaryE8LatticePacker,
    _get_packer_for_bitrate,
    _get_root_e8_lut,
    _FusedE8GEMMFunction,
    _get_ternary_e8_luts,
    fwht_block32,
    pack_model_e8,
)
from .streaming import StreamingE8LoadReport, load_hf_checkpoint_e8, pack_weight_rowwise

__version__ = "0.1.0"

__all__ = [
    "grouped",
    "hardware",
    "ops",
    "optim_state",
    "E8LatticeLinear",
    "E8QuantizationAwareLinear",
    "_E8STEFunction",
    "conway_sloane_e8_project",
    "fast_walsh_hadamard_transform",
    "randomized_hadamard_transform",
    "E8LatticePacker",
    "RootE8LatticePacker",
    "TernaryE8LatticePacker",
    "_get_packer_for_bitrate",
    "_get_root_e8_lut",
    "_FusedE8GEMMFunction",
    "_get_ternary_e8_luts",
    "fwht_block32",
    "pack_model_e8",
    "pack_weight_rowwise",
    "load_hf_checkpoint_e8",
    "StreamingE8LoadReport",
]
