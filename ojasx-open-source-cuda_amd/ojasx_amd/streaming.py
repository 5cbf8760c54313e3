"""Row-block packing and checkpoint-direct loading with the reference's layout contract
(ojasx2/streaming_e8.py).

``pack_weight_rowwise`` packs ``row_block`` rows at a time and returns bytes
identical to whole-matrix packing whenever every row holds whole groups
(``in_features % group_size == 0``); layouts that would let a group cross a row
are rejected with the reference's ``ValueError`` messages.

``load_hf_checkpoint_e8`` builds a Hugging Face causal LM on meta tensors, replaces its
linears by E8 layers and fills their packed buffers from safetensors row blocks
(streaming_e8.py:255-558).  Each row block goes to the GPU and is encoded by the HIP
encoder straight into that layer's packed image in device memory (rows own whole groups,
so the bytes are those of whole-matrix packing); the image is copied to the layer's
buffers once per tensor.  The loaded model keeps the reference's contract: base weights
frozen, LoRA adapters trainable, buffers on the CPU (move the model to the GPU to run the
fused forward).
"""

from __future__ import annotations

import fnmatch
import json
import logging
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Dict, Iterable, List, Sequence, Set, Tuple

import torch
from torch import nn

from . import _native as N
from .lattice import E8LatticeLinear, _get_packer_for_bitrate, _on_gpu, fwht_block32

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


# --------------------------------------------------------------------------- checkpoint-direct load

_LOGGER = logging.getLogger(__name__)


@dataclass(frozen=True)
class StreamingE8LoadReport:
    """Persistent-tensor ledger of a checkpoint-direct load (streaming_e8.py:43-75): the
    same fields, meaning and ``to_dict``; not RSS and not a training peak."""

    checkpoint_dir: str
    architectures: Tuple[str, ...]
    bitrate: float
    group_size: int
    lora_rank: int
    row_block: int
    checkpoint_files: Tuple[str, ...]
    quantized_linear_layers: int
    quantized_source_parameters: int
    packed_weight_bytes: int
    packed_scale_bytes: int
    parameter_bytes: int
    other_buffer_bytes: int
    estimated_persistent_tensor_bytes: int
    trainable_parameters: int
    trainable_parameter_bytes: int
    dense_source_parameters: int
    max_source_row_block_bytes: int
    ignored_checkpoint_keys: Tuple[str, ...]
    memory_scope: str = (
        "persistent tensors only; excludes RSS, Python/allocator overhead, "
        "activations, autograd tape, gradients, optimizer state, and workspaces"
    )

    def to_dict(self) -> Dict[str, object]:
        return asdict(self)


def _checkpoint_files(root: Path) -> Tuple[Path, ...]:
    """The shard list (streaming_e8.py:226-252): the index's weight_map, else
    model.safetensors, else every *.safetensors; shards must exist inside root."""
    index = root / "model.safetensors.index.json"
    if index.is_file():
        with index.open("r", encoding="utf-8") as fh:
            weight_map = json.load(fh).get("weight_map")
        if not isinstance(weight_map, dict) or not weight_map:
            raise ValueError(f"Invalid or empty weight_map in {index}")
        files = tuple(root / name for name in sorted({str(v) for v in weight_map.values()}))
    elif (root / "model.safetensors").is_file():
        files = (root / "model.safetensors",)
    else:
        files = tuple(sorted(root.glob("*.safetensors")))
    if not files:
        raise FileNotFoundError(f"No safetensors checkpoint found under {root}")
    for f in files:
        if not f.is_file():
            raise FileNotFoundError(f"Checkpoint index references missing file: {f}")
        if f.resolve().parent != root.resolve():
            raise ValueError("Checkpoint shard paths must remain inside the checkpoint directory")
    return files


_ENCODERS = {1.5: "ojx_e8t_encode", 2.0: "ojx_e8_encode", 1.0: "ojx_e8r_encode"}
_BITS_PER_16 = {1.5: 3, 2.0: 4, 1.0: 2}  # packed bytes per 16 weights


class _PackedImage:
    """One E8 layer's packed buffers in device memory, filled row block by row block by the
    HIP encoder and copied into the layer's own buffers once complete."""

    def __init__(self, layer: E8LatticeLinear, device: torch.device):
        self.layer = layer
        self.bitrate = float(layer.bitrate)
        self.gs = int(layer.group_size)
        k = int(layer.in_features)
        self.row_bytes = k * _BITS_PER_16[self.bitrate] // 16
        self.row_scales = k // self.gs
        self.device = device
        self.packed = torch.empty(layer.packed_weight.numel(), dtype=torch.uint8, device=device)
        self.scales = torch.empty(layer.block_scales.numel(), dtype=torch.float16, device=device)
        self.rows_done = 0

    def encode(self, row_start: int, block: torch.Tensor, use_hadamard: bool) -> None:
        rows = int(block.shape[0])
        dst_b = row_start * self.row_bytes
        dst_s = row_start * self.row_scales
        if dst_b + rows * self.row_bytes > self.packed.numel():
            raise RuntimeError("Packed destination is smaller than the streamed source layout")
        if dst_s + rows * self.row_scales > self.scales.numel():
            raise RuntimeError("Scale destination is smaller than the streamed source layout")
        src = block.to(self.device, non_blocking=False)
        if src.dtype not in N.DTYPE_CODE:
            src = src.to(torch.float32)
        if use_hadamard:
            src = fwht_block32(src)
        src = src.contiguous()
        with torch.cuda.device(self.device):
            fn = getattr(N.lib(), _ENCODERS[self.bitrate])
            N.check(fn(N.ptr(src), N.DTYPE_CODE[src.dtype], src.numel(), self.gs,
                       self.packed.data_ptr() + dst_b, self.scales.data_ptr() + 2 * dst_s,
                       N.stream_handle(self.device)), "streamed row-block encode")
        self.rows_done += rows

    def commit(self) -> None:
        with torch.no_grad():
            self.layer.packed_weight.copy_(self.packed)
            self.layer.block_scales.copy_(self.scales)


def _stream_weight(handle, key: str, layer: E8LatticeLinear, row_block: int,
                   use_hadamard: bool, device: torch.device) -> int:
    """Reads tensor ``key`` in row blocks (safetensors slices) and packs it into ``layer``
    (streaming_e8.py:161-214); returns the largest block's source bytes."""
    source = handle.get_slice(key)
    shape = tuple(int(d) for d in source.get_shape())
    expected = (int(layer.out_features), int(layer.in_features))
    if shape != expected:
        raise ValueError(f"Checkpoint tensor {key!r} has shape {shape}, expected {expected}")
    image = _PackedImage(layer, device)
    largest = 0
    for start in range(0, expected[0], row_block):
        block = source[start:min(start + row_block, expected[0])]
        if block.ndim != 2 or block.shape[1] != layer.in_features:
            raise ValueError(f"Unexpected row block shape {tuple(block.shape)} for "
                             f"{layer.out_features}x{layer.in_features} E8 layer")
        if not block.dtype.is_floating_point:
            raise TypeError(f"E8 packing requires floating-point source weights, got {block.dtype}")
        image.encode(start, block, use_hadamard)
        largest = max(largest, int(block.numel() * block.element_size()))
        del block
    image.commit()
    return largest


def _matches_any(name: str, patterns: Sequence[str]) -> bool:
    return any(fnmatch.fnmatchcase(name, p) for p in patterns)


def _resolve(model: nn.Module, dotted: str):
    parent = model
    *path, leaf = dotted.split(".")
    for part in path:
        parent = getattr(parent, part)
    return parent, leaf


def load_hf_checkpoint_e8(checkpoint_dir: str, *, bitrate: float = 1.5, group_size: int = 32,
                          lora_rank: int = 8, lora_alpha: float = 16.0, row_block: int = 32,
                          use_hadamard: bool = False, adapter_dtype: torch.dtype = torch.float32,
                          exclude_modules: Iterable[str] = (),
                          allow_unexpected_keys: bool = False
                          ) -> Tuple[nn.Module, StreamingE8LoadReport]:
    """Builds a Hugging Face causal LM from a local checkpoint without materialising dense
    linears (streaming_e8.py:255-558): same arguments, checks, errors and report.

    Every selected nn.Linear becomes an E8LatticeLinear before ingestion; its weight is read
    in ``row_block``-row slices and encoded on the current GPU into the packed buffers;
    other tensors are assigned one shard at a time.  Tied weights of a selected linear,
    missing, duplicate or unexpected tensors and residual meta tensors are errors.  Base
    parameters end frozen; only the LoRA adapters are trainable."""
    if row_block <= 0:
        raise ValueError("row_block must be positive")
    if lora_rank < 0:
        raise ValueError("lora_rank must be non-negative")
    if float(bitrate) not in _SUPPORTED_BITRATES:
        raise ValueError(f"Unsupported E8 bitrate {bitrate!r}; expected one of "
                         f"{sorted(_SUPPORTED_BITRATES)}")
    if group_size <= 0 or group_size % 32 != 0:
        raise ValueError("group_size must be a positive multiple of 32")
    root = Path(checkpoint_dir).expanduser().resolve()
    if not root.is_dir():
        raise NotADirectoryError(f"Local checkpoint directory does not exist: {root}")
    try:
        from accelerate import init_empty_weights
        from safetensors import safe_open
        from transformers import AutoConfig, AutoModelForCausalLM
    except ImportError as exc:
        raise ImportError("Checkpoint-direct E8 loading requires the 'streaming' optional "
                          "dependencies: transformers, accelerate, and safetensors") from exc
    device = _on_gpu(torch.empty(0)).device  # the encoder's device (raises without a GPU)

    files = _checkpoint_files(root)
    config = AutoConfig.from_pretrained(str(root), local_files_only=True,
                                        trust_remote_code=False)
    with init_empty_weights(include_buffers=False):
        model = AutoModelForCausalLM.from_config(config, trust_remote_code=False)
    model.tie_weights()

    excluded = tuple(exclude_modules)
    selected = {name for name, mod in model.named_modules()
                if isinstance(mod, nn.Linear) and not _matches_any(name, excluded)}
    owners: Dict[int, List[str]] = {}
    for name, param in model.named_parameters(remove_duplicate=False):
        owners.setdefault(id(param), []).append(name)
    shared = [names for names in owners.values() if len(names) > 1]
    selected_weights = {f"{n}.weight" for n in selected}
    for names in shared:
        if any(n in selected_weights for n in names):
            raise ValueError("A selected E8 linear shares its weight with another module: "
                             + ", ".join(names) + ". Independent packing would break weight "
                             "tying. Exclude the tied head/module explicitly, or add a "
                             "separately validated tying policy.")

    weight_layers: Dict[str, E8LatticeLinear] = {}
    bias_layers: Dict[str, E8LatticeLinear] = {}
    quantized_params = 0
    for name in sorted(selected, key=lambda n: n.count(".")):
        parent, leaf = _resolve(model, name)
        dense = getattr(parent, leaf)
        _validate_row_layout(int(dense.out_features), int(dense.in_features), float(bitrate),
                             int(group_size))
        layer = E8LatticeLinear(int(dense.in_features), int(dense.out_features),
                                bias=dense.bias is not None, rank=int(lora_rank),
                                lora_alpha=float(lora_alpha), bitrate=float(bitrate),
                                group_size=int(group_size), use_hadamard=bool(use_hadamard),
                                device=torch.device("cpu"), dtype=adapter_dtype)
        setattr(parent, leaf, layer)
        weight_layers[f"{name}.weight"] = layer
        if layer.bias is not None:
            layer.bias.requires_grad_(False)
            bias_layers[f"{name}.bias"] = layer
        quantized_params += int(dense.in_features) * int(dense.out_features)
    if not weight_layers:
        raise ValueError("No eligible nn.Linear modules were selected for E8 conversion")

    state_keys = set(model.state_dict())
    converted = {f"{k[:-len('.weight')]}.{suffix}" for k in weight_layers
                 for suffix in ("packed_weight", "block_scales", "lora_A", "lora_B")}
    tied_keys = {n for names in shared for n in names}
    expected_dense = state_keys - converted - tied_keys
    expected_packed = set(weight_layers) | set(bias_layers)
    seen: Set[str] = set()
    ignored: List[str] = []
    largest_block = 0
    dense_params = 0
    for f in files:
        _LOGGER.info("Streaming checkpoint shard %s", f.name)
        dense_tensors: Dict[str, torch.Tensor] = {}
        with safe_open(str(f), framework="pt", device="cpu") as handle:
            for key in handle.keys():
                if key in seen:
                    raise ValueError(f"Duplicate checkpoint tensor across shards: {key}")
                seen.add(key)
                if key in weight_layers:
                    largest_block = max(largest_block, _stream_weight(
                        handle, key, weight_layers[key], int(row_block), bool(use_hadamard),
                        device))
                elif key in bias_layers:
                    layer = bias_layers[key]
                    t = handle.get_tensor(key)
                    if tuple(t.shape) != (int(layer.out_features),):
                        raise ValueError(f"Unexpected bias shape for {key}: {tuple(t.shape)}")
                    with torch.no_grad():
                        layer.bias.copy_(t)
                    dense_params += int(t.numel())
                elif key in state_keys:
                    dense_tensors[key] = handle.get_tensor(key)
                    dense_params += int(dense_tensors[key].numel())
                elif allow_unexpected_keys:
                    ignored.append(key)
                else:
                    raise ValueError(f"Unexpected checkpoint tensor {key!r} in {f.name}; "
                                     "refusing a silent partial load")
        if dense_tensors:
            model.load_state_dict(dense_tensors, strict=False, assign=True)
            dense_tensors.clear()

    missing = sorted(expected_packed - seen)
    if missing:
        raise ValueError("Checkpoint is missing tensors required by converted E8 layers: "
                         + ", ".join(missing[:20]))
    missing = sorted(expected_dense - seen)
    if missing:
        raise ValueError("Checkpoint is missing required dense parameters or persistent "
                         "buffers: " + ", ".join(missing[:20]))
    for names in shared:
        if not any(n in seen for n in names):
            raise ValueError("Checkpoint contains no stored tensor for shared parameter "
                             "group: " + ", ".join(names))
        # safetensors usually stores one member of a tied group: re-tie to it
        members = [getattr(*_resolve(model, n)) for n in names]
        real = next((p for p in members if not p.is_meta), None)
        if real is not None:
            for n in names:
                parent, leaf = _resolve(model, n)
                setattr(parent, leaf, real)
    residual = [n for n, p in model.named_parameters() if p.is_meta]
    residual += [n for n, b in model.named_buffers() if b.is_meta]
    if residual:
        raise ValueError("Checkpoint load left uninitialized meta tensors: "
                         + ", ".join(residual[:30]))

    for p in model.parameters():
        p.requires_grad_(False)
    for layer in weight_layers.values():
        if layer.lora_A is not None and layer.lora_A.numel():
            layer.lora_A.requires_grad_(True)
            layer.lora_B.requires_grad_(True)

    params = list(model.parameters())
    parameter_bytes = sum(int(p.numel() * p.element_size()) for p in params)
    trainable = [p for p in params if p.requires_grad]
    packed_bytes = sum(int(l.packed_weight.numel()) for l in weight_layers.values())
    scale_bytes = sum(int(l.block_scales.numel() * l.block_scales.element_size())
                      for l in weight_layers.values())
    packed_ids = {id(b) for l in weight_layers.values() for b in (l.packed_weight, l.block_scales)}
    other_bytes = sum(int(b.numel() * b.element_size()) for b in model.buffers()
                      if id(b) not in packed_ids)
    report = StreamingE8LoadReport(
        checkpoint_dir=str(root),
        architectures=tuple(getattr(config, "architectures", ()) or (type(model).__name__,)),
        bitrate=float(bitrate), group_size=int(group_size), lora_rank=int(lora_rank),
        row_block=int(row_block), checkpoint_files=tuple(f.name for f in files),
        quantized_linear_layers=len(weight_layers), quantized_source_parameters=quantized_params,
        packed_weight_bytes=packed_bytes, packed_scale_bytes=scale_bytes,
        parameter_bytes=parameter_bytes, other_buffer_bytes=other_bytes,
        estimated_persistent_tensor_bytes=parameter_bytes + packed_bytes + scale_bytes + other_bytes,
        trainable_parameters=sum(int(p.numel()) for p in trainable),
        trainable_parameter_bytes=sum(int(p.numel() * p.element_size()) for p in trainable),
        dense_source_parameters=dense_params, max_source_row_block_bytes=largest_block,
        ignored_checkpoint_keys=tuple(sorted(ignored)))
    model.ojasx_streaming_report = report
    return model, report
