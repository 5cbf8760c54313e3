"""``torch.library`` custom ops (namespace ``ojasx_e8t``) over the C ABI.

Ops and the reference interfaces they replace:

* ``encode(w, group_size) -> (packed, scales)``
    TernaryE8LatticePacker.pack (ojasx2/math/lattice.py:338-384)
* ``decode(packed, scales, numel, group_size, dtype) -> W``
    TernaryE8LatticePacker.unpack (lattice.py:386-419)
* ``e8t_linear(x, packed_weight, block_scales, bias, out_features, in_features,
  group_size) -> y``  (autograd registered; saves only packed and scales, as
  lattice.py:569 does)
    the routing of _FusedE8GEMMFunction.forward/backward (lattice.py:552-717)
    with the TileLang / native / portable backends replaced by one HIP path
* ``fused_ternary_e8_gemm_fwd`` / ``fused_ternary_e8_gemm_bwd_dx``
    the reference's native op schemas (ojasx_math_bindings.cpp:593-594) with the
    binding's layout checks (:17-34, :414-433), for callers that bind the op by name.
* 2-bit E8 (E8LatticePacker, lattice.py:209-279): ``encode2`` / ``decode2``,
  ``e8_linear`` (autograd) / ``e8_linear_bwd_dx``, and the native schemas
  ``fused_e8_gemm_fwd`` / ``fused_e8_gemm_bwd_dx`` (ojasx_math_bindings.cpp:591-592).

Every op runs on the current HIP stream of the input's device, allocates its
outputs through torch's caching allocator and raises ``RuntimeError`` for
unsupported layouts or non-ROCm tensors; nothing silently declines or falls back.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _native as N

_NS = "ojasx_e8t"


def _dtype_code(dt: torch.dtype) -> int:
    try:
        return N.DTYPE_CODE[dt]
    except KeyError:
        raise RuntimeError(f"ojasx_e8t supports float32, float16 and bfloat16 (got {dt})")


def _padded(numel: int, gs: int) -> int:
    return numel + ((-numel) % gs)


def _check_gs(gs: int) -> None:
    if gs <= 0 or gs % 16 != 0:
        raise RuntimeError(f"group_size must be a positive multiple of 16 (got {gs})")


# ----------------------------------------------------------------------------- encode

@torch.library.custom_op(f"{_NS}::encode", mutates_args=())
def encode(w: torch.Tensor, group_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    dev = N.require_device(w)
    _check_gs(group_size)
    if w.dtype not in N.DTYPE_CODE:
        w = w.to(torch.float32)  # the reference widens to fp32 first (lattice.py:350)
    w = w.contiguous()
    numel = w.numel()
    padded = _padded(numel, group_size)
    packed = torch.empty(padded * 3 // 16, dtype=torch.uint8, device=dev)
    scales = torch.empty(padded // group_size, dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        N.check(N.lib().ojx_e8t_encode(N.ptr(w), _dtype_code(w.dtype), numel, group_size,
                                       N.ptr(packed), N.ptr(scales), N.stream_handle(dev)),
                "encode")
    return packed, scales


@encode.register_fake
def _(w, group_size):
    padded = _padded(w.numel(), group_size)
    return (w.new_empty(padded * 3 // 16, dtype=torch.uint8),
            w.new_empty(padded // group_size, dtype=torch.float16))


# ----------------------------------------------------------------------------- decode

@torch.library.custom_op(f"{_NS}::decode", mutates_args=())
def decode(packed: torch.Tensor, scales: torch.Tensor, numel: int, group_size: int,
           dtype: torch.dtype) -> torch.Tensor:
    dev = N.require_device(packed, scales)
    _check_gs(group_size)
    if packed.dtype != torch.uint8 or scales.dtype != torch.float16:
        raise RuntimeError("decode expects uint8 packed codes and float16 scales")
    padded = _padded(numel, group_size)
    if packed.numel() < padded * 3 // 16 or scales.numel() < padded // group_size:
        raise RuntimeError(
            f"packed/scales too small for {numel} weights at group_size {group_size}")
    packed = packed.contiguous()
    scales = scales.contiguous()
    out = torch.empty(numel, dtype=dtype, device=dev)
    with torch.cuda.device(dev):
        N.check(N.lib().ojx_e8t_decode(N.ptr(packed), N.ptr(scales), numel, group_size,
                                       _dtype_code(dtype), N.ptr(out), N.stream_handle(dev)),
                "decode")
    return out


@decode.register_fake
def _(packed, scales, numel, group_size, dtype):
    return packed.new_empty(numel, dtype=dtype)


# ----------------------------------------------------------------------------- linear

def _check_layer_buffers(packed: torch.Tensor, scales: torch.Tensor, out_features: int,
                         in_features: int, group_size: int) -> None:
    if packed.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    if not scales.is_floating_point():
        raise RuntimeError("block_scales must be a floating-point tensor (float16 bits)")
    padded = _padded(out_features * in_features, group_size)
    if packed.numel() < padded * 3 // 16:
        raise RuntimeError(
            f"packed_weight holds {packed.numel()} bytes; {out_features}x{in_features} at "
            f"group_size {group_size} needs {padded * 3 // 16}")
    if scales.numel() < padded // group_size:
        raise RuntimeError(
            f"block_scales holds {scales.numel()} values; needs {padded // group_size}")


FMT_TERNARY, FMT_E8, FMT_ROOT = 0, 1, 2
_FWD = {FMT_TERNARY: "ojx_e8t_gemm_fwd", FMT_E8: "ojx_e8_gemm_fwd", FMT_ROOT: "ojx_e8r_gemm_fwd"}
_BWD = {FMT_TERNARY: "ojx_e8t_gemm_bwd_dx", FMT_E8: "ojx_e8_gemm_bwd_dx",
        FMT_ROOT: "ojx_e8r_gemm_bwd_dx"}


def workspace(fmt: int, bwd: bool, M: int, N_out: int, K: int, group_size: int,
              dtype: torch.dtype, device: torch.device) -> Optional[torch.Tensor]:
    """The scratch a fused GEMM launch uses (``ojx_gemm_workspace_bytes``), from torch's
    caching allocator, or None when the launch needs none.  Allocated per call, so a launch
    captured into a CUDA graph keeps its workspace in the graph's memory pool."""
    nbytes = ctypes.c_size_t(0)
    N.check(N.lib().ojx_gemm_workspace_bytes(fmt, int(bwd), M, N_out, K, group_size,
                                             _dtype_code(dtype), ctypes.byref(nbytes)),
            "gemm_workspace_bytes")
    if nbytes.value == 0:
        return None
    return torch.empty(nbytes.value, dtype=torch.uint8, device=device)


def _linear_fwd(fmt: int, x: torch.Tensor, packed_weight: torch.Tensor,
                block_scales: torch.Tensor, bias: Optional[torch.Tensor], out_features: int,
                in_features: int, group_size: int) -> torch.Tensor:
    """y = x . Wdeq^T (+ bias) through the format's fused forward.  Every buffer handed to
    the library is bound to a local that lives until the launch has been enqueued."""
    dev = N.require_device(x, packed_weight, block_scales, bias)
    dt = _dtype_code(x.dtype)
    x2 = x.reshape(-1, in_features).contiguous()
    M = x2.shape[0]
    y = torch.empty((M, out_features), dtype=x.dtype, device=dev)
    b = None
    if bias is not None:
        if bias.numel() != out_features:
            raise RuntimeError(f"bias has {bias.numel()} elements, expected {out_features}")
        b = bias.to(x.dtype).contiguous()  # the reference casts bias to x's dtype
    pw = packed_weight.contiguous()
    # the buffer holds fp16 scales; a module cast (e.g. .to(bfloat16)) leaves them in another
    # float dtype, which the reference tolerates (scales.to(dtype), lattice.py:414-418)
    bs = block_scales.to(torch.float16).contiguous()
    with torch.cuda.device(dev):
        ws = workspace(fmt, False, M, out_features, in_features, group_size, x.dtype, dev)
        N.check(getattr(N.lib(), _FWD[fmt])(N.ptr(x2), N.ptr(pw), N.ptr(bs), N.ptr(b), N.ptr(y),
                                            M, out_features, in_features, group_size, dt,
                                            N.ptr(ws), 0 if ws is None else ws.numel(),
                                            N.stream_handle(dev)),
                _FWD[fmt][4:])
    return y.reshape(*x.shape[:-1], out_features)


def _linear_bwd(fmt: int, grad_y: torch.Tensor, packed_weight: torch.Tensor,
                block_scales: torch.Tensor, out_features: int, in_features: int,
                group_size: int) -> torch.Tensor:
    """grad_x = grad_y . Wdeq through the format's fused backward dX."""
    dev = N.require_device(grad_y, packed_weight, block_scales)
    if grad_y.shape[-1] != out_features:
        raise RuntimeError(f"grad_y has {grad_y.shape[-1]} features, expected {out_features}")
    dt = _dtype_code(grad_y.dtype)
    gy = grad_y.reshape(-1, out_features).contiguous()
    M = gy.shape[0]
    gx = torch.empty((M, in_features), dtype=grad_y.dtype, device=dev)
    pw = packed_weight.contiguous()
    # the buffer holds fp16 scales; a module cast (e.g. .to(bfloat16)) leaves them in another
    # float dtype, which the reference tolerates (scales.to(dtype), lattice.py:414-418)
    bs = block_scales.to(torch.float16).contiguous()
    with torch.cuda.device(dev):
        ws = workspace(fmt, True, M, out_features, in_features, group_size, grad_y.dtype, dev)
        N.check(getattr(N.lib(), _BWD[fmt])(N.ptr(gy), N.ptr(pw), N.ptr(bs), N.ptr(gx), M,
                                            out_features, in_features, group_size, dt,
                                            N.ptr(ws), 0 if ws is None else ws.numel(),
                                            N.stream_handle(dev)),
                _BWD[fmt][4:])
    return gx.reshape(*grad_y.shape[:-1], in_features)


@torch.library.custom_op(f"{_NS}::e8t_linear", mutates_args=())
def e8t_linear(x: torch.Tensor, packed_weight: torch.Tensor, block_scales: torch.Tensor,
               bias: Optional[torch.Tensor], out_features: int, in_features: int,
               group_size: int) -> torch.Tensor:
    N.require_device(x, packed_weight, block_scales, bias)
    _check_gs(group_size)
    if x.shape[-1] != in_features:
        raise RuntimeError(f"x has {x.shape[-1]} features, layer expects {in_features}")
    _check_layer_buffers(packed_weight, block_scales, out_features, in_features, group_size)
    return _linear_fwd(FMT_TERNARY, x, packed_weight, block_scales, bias, out_features,
                       in_features, group_size)


@e8t_linear.register_fake
def _(x, packed_weight, block_scales, bias, out_features, in_features, group_size):
    return x.new_empty((*x.shape[:-1], out_features))


@torch.library.custom_op(f"{_NS}::e8t_linear_bwd_dx", mutates_args=())
def e8t_linear_bwd_dx(grad_y: torch.Tensor, packed_weight: torch.Tensor,
                      block_scales: torch.Tensor, out_features: int, in_features: int,
                      group_size: int) -> torch.Tensor:
    N.require_device(grad_y, packed_weight, block_scales)
    _check_gs(group_size)
    _check_layer_buffers(packed_weight, block_scales, out_features, in_features, group_size)
    return _linear_bwd(FMT_TERNARY, grad_y, packed_weight, block_scales, out_features,
                       in_features, group_size)


@e8t_linear_bwd_dx.register_fake
def _(grad_y, packed_weight, block_scales, out_features, in_features, group_size):
    return grad_y.new_empty((*grad_y.shape[:-1], in_features))


def _linear_setup_context(ctx, inputs, output):
    x, packed_weight, block_scales, bias, out_features, in_features, group_size = inputs
    ctx.save_for_backward(packed_weight, block_scales)
    ctx.dims = (out_features, in_features, group_size)
    ctx.has_bias = bias is not None


def _linear_backward(ctx, grad_y):
    packed_weight, block_scales = ctx.saved_tensors
    out_features, in_features, group_size = ctx.dims
    grad_x = None
    if ctx.needs_input_grad[0]:
        grad_x = e8t_linear_bwd_dx(grad_y, packed_weight, block_scales, out_features,
                                   in_features, group_size)
    grad_bias = grad_y.reshape(-1, out_features).sum(dim=0) if ctx.has_bias else None
    return grad_x, None, None, grad_bias, None, None, None


e8t_linear.register_autograd(_linear_backward, setup_context=_linear_setup_context)


# ----------------------------------------------------------- fused LoRA epilogue

_FWD_LORA = {FMT_TERNARY: "ojx_e8t_gemm_fwd_lora", FMT_E8: "ojx_e8_gemm_fwd_lora",
             FMT_ROOT: "ojx_e8r_gemm_fwd_lora"}
LORA_MAX_RANK = 64  # ojx_lora_down's rank range (include/ojasx_e8t.h)


def _check_fmt_layer(fmt: int, packed_weight: torch.Tensor, block_scales: torch.Tensor,
                     out_features: int, in_features: int, group_size: int) -> None:
    if fmt == FMT_TERNARY:
        _check_gs(group_size)
        _check_layer_buffers(packed_weight, block_scales, out_features, in_features, group_size)
    elif fmt == FMT_E8:
        _check_gs2(group_size, 4)
        _check_layer_buffers2(packed_weight, block_scales, out_features, in_features, group_size)
    elif fmt == FMT_ROOT:
        _check_gs2(group_size, 8)
        _check_layer_buffers1(packed_weight, block_scales, out_features, in_features, group_size)
    else:
        raise RuntimeError(f"unknown weight format {fmt}")


@torch.library.custom_op(f"{_NS}::linear_lora", mutates_args=())
def linear_lora(x: torch.Tensor, packed_weight: torch.Tensor, block_scales: torch.Tensor,
                bias: Optional[torch.Tensor], lora_a: torch.Tensor, lora_b: torch.Tensor,
                scaling: float, fmt: int, out_features: int, in_features: int,
                group_size: int) -> torch.Tensor:
    """x . Wdeq^T (+ bias) + scaling * (x @ lora_a) @ lora_b in one fused forward: the E8
    op and E8LatticeLinear's adapter term (lattice.py:839-842), lora_a [in, r] and lora_b
    [r, out] in x's dtype, the adapter term added in fp32 in the E8 kernel's epilogue."""
    dev = N.require_device(x, packed_weight, block_scales, bias, lora_a, lora_b)
    if x.shape[-1] != in_features:
        raise RuntimeError(f"x has {x.shape[-1]} features, layer expects {in_features}")
    _check_fmt_layer(fmt, packed_weight, block_scales, out_features, in_features, group_size)
    r = lora_a.shape[-1]
    if lora_a.dim() != 2 or lora_a.shape[0] != in_features or tuple(lora_b.shape) != (r, out_features):
        raise RuntimeError(f"LoRA factors must be [{in_features}, r] and [r, {out_features}] "
                           f"(got {tuple(lora_a.shape)} and {tuple(lora_b.shape)})")
    if not 1 <= r <= LORA_MAX_RANK:
        raise RuntimeError(f"fused LoRA supports ranks 1..{LORA_MAX_RANK} (got {r})")
    dt = _dtype_code(x.dtype)
    x2 = x.reshape(-1, in_features).contiguous()
    M = x2.shape[0]
    y = torch.empty((M, out_features), dtype=x.dtype, device=dev)
    b = None
    if bias is not None:
        if bias.numel() != out_features:
            raise RuntimeError(f"bias has {bias.numel()} elements, expected {out_features}")
        b = bias.to(x.dtype).contiguous()
    la = lora_a.to(x.dtype).contiguous()
    lb = lora_b.to(x.dtype).contiguous()
    pw = packed_weight.contiguous()
    # the buffer holds fp16 scales; a module cast (e.g. .to(bfloat16)) leaves them in another
    # float dtype, which the reference tolerates (scales.to(dtype), lattice.py:414-418)
    bs = block_scales.to(torch.float16).contiguous()
    u = torch.empty((M, r), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        ws = workspace(fmt, False, M, out_features, in_features, group_size, x.dtype, dev)
        N.check(getattr(N.lib(), _FWD_LORA[fmt])(
            N.ptr(x2), N.ptr(pw), N.ptr(bs), N.ptr(b), N.ptr(la), N.ptr(lb), r, float(scaling),
            N.ptr(u), N.ptr(y), M, out_features, in_features, group_size, dt, N.ptr(ws),
            0 if ws is None else ws.numel(), N.stream_handle(dev)),
            _FWD_LORA[fmt][4:])
    return y.reshape(*x.shape[:-1], out_features)


@linear_lora.register_fake
def _(x, packed_weight, block_scales, bias, lora_a, lora_b, scaling, fmt, out_features,
      in_features, group_size):
    return x.new_empty((*x.shape[:-1], out_features))


def _linear_lora_setup_context(ctx, inputs, output):
    (x, packed_weight, block_scales, bias, lora_a, lora_b, scaling, fmt, out_features,
     in_features, group_size) = inputs
    ctx.save_for_backward(x, packed_weight, block_scales, lora_a, lora_b)
    ctx.dims = (out_features, in_features, group_size)
    ctx.fmt = fmt
    ctx.scaling = float(scaling)
    ctx.has_bias = bias is not None
    ctx.bias_dtype = None if bias is None else bias.dtype


def _linear_lora_backward(ctx, grad_y):
    """grad_x through the fused backward dX plus the adapter's term; the adapter's own
    gradients (and the bias's) in torch, as the reference computes them."""
    x, packed_weight, block_scales, lora_a, lora_b = ctx.saved_tensors
    out_features, in_features, group_size = ctx.dims
    sc = ctx.scaling
    gy = grad_y.reshape(-1, out_features).contiguous()
    x2 = x.reshape(-1, in_features)
    la = lora_a.to(grad_y.dtype)
    lb = lora_b.to(grad_y.dtype)
    gyb = gy @ lb.t().contiguous()                       # [M, r]
    grad_x = grad_a = grad_b = grad_bias = None
    if ctx.needs_input_grad[0]:
        grad_x = _linear_bwd(ctx.fmt, gy, packed_weight, block_scales, out_features,
                             in_features, group_size)
        grad_x = (grad_x + sc * (gyb @ la.t().contiguous())).reshape(x.shape)
    if ctx.needs_input_grad[4]:
        grad_a = (sc * (x2.t().contiguous() @ gyb)).to(lora_a.dtype)
    if ctx.needs_input_grad[5]:
        grad_b = (sc * ((x2 @ la).t().contiguous() @ gy)).to(lora_b.dtype)
    if ctx.has_bias and ctx.needs_input_grad[3]:
        grad_bias = gy.sum(dim=0).to(ctx.bias_dtype)
    return grad_x, None, None, grad_bias, grad_a, grad_b, None, None, None, None, None


linear_lora.register_autograd(_linear_lora_backward, setup_context=_linear_lora_setup_context)


# ------------------------------------------------------- reference native op schemas

@torch.library.custom_op(f"{_NS}::fused_ternary_e8_gemm_fwd", mutates_args=())
def fused_ternary_e8_gemm_fwd(x: torch.Tensor, packed_weight: torch.Tensor,
                              block_scales: torch.Tensor, bias: Optional[torch.Tensor] = None,
                              group_size: int = 32) -> torch.Tensor:
    """Same schema and checks as the reference's native op (ojasx_math_bindings.cpp:407-433)."""
    if packed_weight.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    if group_size <= 0 or group_size % 16 != 0:
        raise RuntimeError("group_size must be a positive multiple of 16")
    if x.dim() < 1:
        raise RuntimeError("input must have a feature axis")
    K = x.shape[-1]
    if packed_weight.dim() != 2:
        raise RuntimeError("packed_weight must be a 2D matrix")
    if K <= 0 or K % 16 != 0 or K % group_size != 0:
        raise RuntimeError("feature count must be divisible by the packing unit and group_size")
    Nf = packed_weight.shape[0]
    if block_scales.numel() != Nf * (K // group_size):
        raise RuntimeError("block_scales must contain exactly N * (K / group_size) elements")
    if packed_weight.shape[1] != (K * 3) // 16:
        raise RuntimeError("packed_weight dim 1 must match (in_features * 3) / 16")
    return e8t_linear(x, packed_weight.reshape(-1), block_scales.reshape(-1).to(torch.float16),
                      bias, Nf, K, group_size)


@fused_ternary_e8_gemm_fwd.register_fake
def _(x, packed_weight, block_scales, bias=None, group_size=32):
    return x.new_empty((*x.shape[:-1], packed_weight.shape[0]))


@torch.library.custom_op(f"{_NS}::fused_ternary_e8_gemm_bwd_dx", mutates_args=())
def fused_ternary_e8_gemm_bwd_dx(grad_y: torch.Tensor, packed_weight: torch.Tensor,
                                 block_scales: torch.Tensor, in_features: int,
                                 group_size: int = 32) -> torch.Tensor:
    """Same schema and checks as the reference's native op (ojasx_math_bindings.cpp:479-500)."""
    if packed_weight.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    if packed_weight.dim() != 2:
        raise RuntimeError("packed_weight must be 2D [N, (K * 3) / 16]")
    if packed_weight.shape[1] != (in_features * 3) // 16:
        raise RuntimeError("packed_weight dim 1 must match (in_features * 3) / 16")
    if group_size <= 0 or group_size % 16 != 0:
        raise RuntimeError("group_size must be a positive multiple of 16")
    K = in_features
    if K <= 0 or K % 16 != 0 or K % group_size != 0:
        raise RuntimeError("feature count must be divisible by the packing unit and group_size")
    Nf = packed_weight.shape[0]
    if block_scales.numel() != Nf * (K // group_size):
        raise RuntimeError("block_scales must contain exactly N * (K / group_size) elements")
    if grad_y.shape[-1] != Nf:
        raise RuntimeError("Last dimension of grad_y must match N")
    return e8t_linear_bwd_dx(grad_y, packed_weight.reshape(-1),
                             block_scales.reshape(-1).to(torch.float16), Nf, K, group_size)


@fused_ternary_e8_gemm_bwd_dx.register_fake
def _(grad_y, packed_weight, block_scales, in_features, group_size=32):
    return grad_y.new_empty((*grad_y.shape[:-1], in_features))


# ----------------------------------------------------------------------------- 2-bit E8

def _check_gs2(gs: int, unit: int) -> None:
    if gs <= 0 or gs % unit != 0:
        raise RuntimeError(f"group_size must be a positive multiple of {unit} (got {gs})")


@torch.library.custom_op(f"{_NS}::encode2", mutates_args=())
def encode2(w: torch.Tensor, group_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """E8LatticePacker.pack (lattice.py:213-249): (packed uint8 [padded/4], fp16 scales)."""
    dev = N.require_device(w)
    _check_gs2(group_size, 8)
    if w.dtype not in N.DTYPE_CODE:
        w = w.to(torch.float32)  # the reference widens to fp32 first (lattice.py:222)
    w = w.contiguous()
    numel = w.numel()
    padded = _padded(numel, group_size)
    packed = torch.empty(padded // 4, dtype=torch.uint8, device=dev)
    scales = torch.empty(padded // group_size, dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        N.check(N.lib().ojx_e8_encode(N.ptr(w), _dtype_code(w.dtype), numel, group_size,
                                      N.ptr(packed), N.ptr(scales), N.stream_handle(dev)),
                "e8 encode")
    return packed, scales


@encode2.register_fake
def _(w, group_size):
    padded = _padded(w.numel(), group_size)
    return (w.new_empty(padded // 4, dtype=torch.uint8),
            w.new_empty(padded // group_size, dtype=torch.float16))


@torch.library.custom_op(f"{_NS}::decode2", mutates_args=())
def decode2(packed: torch.Tensor, scales: torch.Tensor, numel: int, group_size: int,
            dtype: torch.dtype) -> torch.Tensor:
    """E8LatticePacker.unpack (lattice.py:252-279), flat, first ``numel`` weights."""
    dev = N.require_device(packed, scales)
    _check_gs2(group_size, 8)
    if packed.dtype != torch.uint8 or scales.dtype != torch.float16:
        raise RuntimeError("decode2 expects uint8 packed codes and float16 scales")
    padded = _padded(numel, group_size)
    if packed.numel() < padded // 4 or scales.numel() < padded // group_size:
        raise RuntimeError(
            f"packed/scales too small for {numel} weights at group_size {group_size}")
    packed = packed.contiguous()
    scales = scales.contiguous()
    out = torch.empty(numel, dtype=dtype, device=dev)
    with torch.cuda.device(dev):
        N.check(N.lib().ojx_e8_decode(N.ptr(packed), N.ptr(scales),
                                      numel, group_size, _dtype_code(dtype), N.ptr(out),
                                      N.stream_handle(dev)),
                "e8 decode")
    return out


@decode2.register_fake
def _(packed, scales, numel, group_size, dtype):
    return packed.new_empty(numel, dtype=dtype)


def _check_layer_buffers2(packed: torch.Tensor, scales: torch.Tensor, out_features: int,
                          in_features: int, group_size: int) -> None:
    if packed.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    if not scales.is_floating_point():
        raise RuntimeError("block_scales must be a floating-point tensor (float16 bits)")
    padded = _padded(out_features * in_features, group_size)
    if packed.numel() < padded // 4:
        raise RuntimeError(
            f"packed_weight holds {packed.numel()} bytes; {out_features}x{in_features} at "
            f"group_size {group_size} needs {padded // 4}")
    if scales.numel() < padded // group_size:
        raise RuntimeError(
            f"block_scales holds {scales.numel()} values; needs {padded // group_size}")


@torch.library.custom_op(f"{_NS}::e8_linear", mutates_args=())
def e8_linear(x: torch.Tensor, packed_weight: torch.Tensor, block_scales: torch.Tensor,
              bias: Optional[torch.Tensor], out_features: int, in_features: int,
              group_size: int) -> torch.Tensor:
    """2-bit fused linear: x . Wdeq^T + bias, Wdeq = (code - 1.5) * scale in x's dtype."""
    N.require_device(x, packed_weight, block_scales, bias)
    _check_gs2(group_size, 4)
    if x.shape[-1] != in_features:
        raise RuntimeError(f"x has {x.shape[-1]} features, layer expects {in_features}")
    _check_layer_buffers2(packed_weight, block_scales, out_features, in_features, group_size)
    return _linear_fwd(FMT_E8, x, packed_weight, block_scales, bias, out_features, in_features,
                       group_size)


@e8_linear.register_fake
def _(x, packed_weight, block_scales, bias, out_features, in_features, group_size):
    return x.new_empty((*x.shape[:-1], out_features))


@torch.library.custom_op(f"{_NS}::e8_linear_bwd_dx", mutates_args=())
def e8_linear_bwd_dx(grad_y: torch.Tensor, packed_weight: torch.Tensor,
                     block_scales: torch.Tensor, out_features: int, in_features: int,
                     group_size: int) -> torch.Tensor:
    N.require_device(grad_y, packed_weight, block_scales)
    _check_gs2(group_size, 4)
    _check_layer_buffers2(packed_weight, block_scales, out_features, in_features, group_size)
    return _linear_bwd(FMT_E8, grad_y, packed_weight, block_scales, out_features, in_features,
                       group_size)


@e8_linear_bwd_dx.register_fake
def _(grad_y, packed_weight, block_scales, out_features, in_features, group_size):
    return grad_y.new_empty((*grad_y.shape[:-1], in_features))


def _linear2_backward(ctx, grad_y):
    packed_weight, block_scales = ctx.saved_tensors
    out_features, in_features, group_size = ctx.dims
    grad_x = None
    if ctx.needs_input_grad[0]:
        grad_x = e8_linear_bwd_dx(grad_y, packed_weight, block_scales, out_features,
                                  in_features, group_size)
    grad_bias = grad_y.reshape(-1, out_features).sum(dim=0) if ctx.has_bias else None
    return grad_x, None, None, grad_bias, None, None, None


e8_linear.register_autograd(_linear2_backward, setup_context=_linear_setup_context)


@torch.library.custom_op(f"{_NS}::fused_e8_gemm_fwd", mutates_args=())
def fused_e8_gemm_fwd(x: torch.Tensor, packed_weight: torch.Tensor, block_scales: torch.Tensor,
                      bias: Optional[torch.Tensor] = None, group_size: int = 32) -> torch.Tensor:
    """Same schema and checks as the reference's native op (ojasx_math_bindings.cpp:274-292)."""
    if packed_weight.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    if group_size <= 0 or group_size % 4 != 0:
        raise RuntimeError("group_size must be a positive multiple of 4")
    if x.dim() < 1:
        raise RuntimeError("input must have a feature axis")
    K = x.shape[-1]
    if packed_weight.dim() != 2:
        raise RuntimeError("packed_weight must be a 2D matrix")
    if K <= 0 or K % 4 != 0 or K % group_size != 0:
        raise RuntimeError("feature count must be divisible by the packing unit and group_size")
    Nf = packed_weight.shape[0]
    if block_scales.numel() != Nf * (K // group_size):
        raise RuntimeError("block_scales must contain exactly N * (K / group_size) elements")
    if packed_weight.shape[1] != K // 4:
        raise RuntimeError("packed_weight dim 1 must match in_features / 4")
    return e8_linear(x, packed_weight.reshape(-1), block_scales.reshape(-1).to(torch.float16),
                     bias, Nf, K, group_size)


@fused_e8_gemm_fwd.register_fake
def _(x, packed_weight, block_scales, bias=None, group_size=32):
    return x.new_empty((*x.shape[:-1], packed_weight.shape[0]))


@torch.library.custom_op(f"{_NS}::fused_e8_gemm_bwd_dx", mutates_args=())
def fused_e8_gemm_bwd_dx(grad_y: torch.Tensor, packed_weight: torch.Tensor,
                         block_scales: torch.Tensor, in_features: int,
                         group_size: int = 32) -> torch.Tensor:
    """Same schema and checks as the reference's native op (ojasx_math_bindings.cpp:346-366)."""
    if packed_weight.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    if packed_weight.dim() != 2:
        raise RuntimeError("packed_weight must be 2D [N, K / 4]")
    if packed_weight.shape[1] != in_features // 4:
        raise RuntimeError("packed_weight dim 1 must match in_features / 4")
    if group_size <= 0 or group_size % 4 != 0:
        raise RuntimeError("group_size must be a positive multiple of 4")
    K = in_features
    if K <= 0 or K % 4 != 0 or K % group_size != 0:
        raise RuntimeError("feature count must be divisible by the packing unit and group_size")
    Nf = packed_weight.shape[0]
    if block_scales.numel() != Nf * (K // group_size):
        raise RuntimeError("block_scales must contain exactly N * (K / group_size) elements")
    if grad_y.shape[-1] != Nf:
        raise RuntimeError("Last dimension of grad_y must match N")
    return e8_linear_bwd_dx(grad_y, packed_weight.reshape(-1),
                            block_scales.reshape(-1).to(torch.float16), Nf, K, group_size)


@fused_e8_gemm_bwd_dx.register_fake
def _(grad_y, packed_weight, block_scales, in_features, group_size=32):
    return grad_y.new_empty((*grad_y.shape[:-1], in_features))


# --------------------------------------------------------------------------- 1-bit Root E8

@torch.library.custom_op(f"{_NS}::encode1", mutates_args=())
def encode1(w: torch.Tensor, group_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """RootE8LatticePacker.pack (lattice.py:473-509): (codes uint8 [padded/8], fp16 scales).
    group_size must already be coerced (a positive multiple of 8)."""
    dev = N.require_device(w)
    _check_gs2(group_size, 8)
    if w.dtype not in N.DTYPE_CODE:
        w = w.to(torch.float32)  # the reference widens to fp32 first (lattice.py:489)
    w = w.contiguous()
    numel = w.numel()
    padded = _padded(numel, group_size)
    codes = torch.empty(padded // 8, dtype=torch.uint8, device=dev)
    scales = torch.empty(padded // group_size, dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        N.check(N.lib().ojx_e8r_encode(N.ptr(w), _dtype_code(w.dtype), numel, group_size,
                                       N.ptr(codes), N.ptr(scales), N.stream_handle(dev)),
                "e8r encode")
    return codes, scales


@encode1.register_fake
def _(w, group_size):
    padded = _padded(w.numel(), group_size)
    return (w.new_empty(padded // 8, dtype=torch.uint8),
            w.new_empty(padded // group_size, dtype=torch.float16))


@torch.library.custom_op(f"{_NS}::decode1", mutates_args=())
def decode1(codes: torch.Tensor, scales: torch.Tensor, numel: int, group_size: int,
            dtype: torch.dtype) -> torch.Tensor:
    """RootE8LatticePacker.unpack (lattice.py:519-533), flat, first ``numel`` weights."""
    dev = N.require_device(codes, scales)
    _check_gs2(group_size, 8)
    if codes.dtype != torch.uint8 or scales.dtype != torch.float16:
        raise RuntimeError("decode1 expects uint8 codes and float16 scales")
    padded = _padded(numel, group_size)
    if codes.numel() < padded // 8 or scales.numel() < padded // group_size:
        raise RuntimeError(
            f"codes/scales too small for {numel} weights at group_size {group_size}")
    codes = codes.contiguous()
    scales = scales.contiguous()
    out = torch.empty(numel, dtype=dtype, device=dev)
    with torch.cuda.device(dev):
        N.check(N.lib().ojx_e8r_decode(N.ptr(codes), N.ptr(scales),
                                       numel, group_size, _dtype_code(dtype), N.ptr(out),
                                       N.stream_handle(dev)),
                "e8r decode")
    return out


@decode1.register_fake
def _(codes, scales, numel, group_size, dtype):
    return codes.new_empty(numel, dtype=dtype)


def _check_layer_buffers1(codes: torch.Tensor, scales: torch.Tensor, out_features: int,
                          in_features: int, group_size: int) -> None:
    if codes.dtype != torch.uint8:
        raise RuntimeError("packed_weight must be uint8")
    if not scales.is_floating_point():
        raise RuntimeError("block_scales must be a floating-point tensor (float16 bits)")
    padded = _padded(out_features * in_features, group_size)
    if codes.numel() < padded // 8:
        raise RuntimeError(
            f"packed_weight holds {codes.numel()} bytes; {out_features}x{in_features} at "
            f"group_size {group_size} needs {padded // 8}")
    if scales.numel() < padded // group_size:
        raise RuntimeError(
            f"block_scales holds {scales.numel()} values; needs {padded // group_size}")


@torch.library.custom_op(f"{_NS}::e8r_linear", mutates_args=())
def e8r_linear(x: torch.Tensor, packed_weight: torch.Tensor, block_scales: torch.Tensor,
               bias: Optional[torch.Tensor], out_features: int, in_features: int,
               group_size: int) -> torch.Tensor:
    """1-bit fused linear: x . Wdeq^T + bias, Wdeq = table[code] * scale in x's dtype."""
    N.require_device(x, packed_weight, block_scales, bias)
    _check_gs2(group_size, 8)
    if x.shape[-1] != in_features:
        raise RuntimeError(f"x has {x.shape[-1]} features, layer expects {in_features}")
    _check_layer_buffers1(packed_weight, block_scales, out_features, in_features, group_size)
    return _linear_fwd(FMT_ROOT, x, packed_weight, block_scales, bias, out_features,
                       in_features, group_size)


@e8r_linear.register_fake
def _(x, packed_weight, block_scales, bias, out_features, in_features, group_size):
    return x.new_empty((*x.shape[:-1], out_features))


@torch.library.custom_op(f"{_NS}::e8r_linear_bwd_dx", mutates_args=())
def e8r_linear_bwd_dx(grad_y: torch.Tensor, packed_weight: torch.Tensor,
                      block_scales: torch.Tensor, out_features: int, in_features: int,
                      group_size: int) -> torch.Tensor:
    N.require_device(grad_y, packed_weight, block_scales)
    _check_gs2(group_size, 8)
    _check_layer_buffers1(packed_weight, block_scales, out_features, in_features, group_size)
    return _linear_bwd(FMT_ROOT, grad_y, packed_weight, block_scales, out_features, in_features,
                       group_size)


@e8r_linear_bwd_dx.register_fake
def _(grad_y, packed_weight, block_scales, out_features, in_features, group_size):
    return grad_y.new_empty((*grad_y.shape[:-1], in_features))


def _linear1_backward(ctx, grad_y):
    packed_weight, block_scales = ctx.saved_tensors
    out_features, in_features, group_size = ctx.dims
    grad_x = None
    if ctx.needs_input_grad[0]:
        grad_x = e8r_linear_bwd_dx(grad_y, packed_weight, block_scales, out_features,
                                   in_features, group_size)
    grad_bias = grad_y.reshape(-1, out_features).sum(dim=0) if ctx.has_bias else None
    return grad_x, None, None, grad_bias, None, None, None


e8r_linear.register_autograd(_linear1_backward, setup_context=_linear_setup_context)


# --------------------------------------------------------------------------- Hadamard rotation

_FWHT_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}


@torch.library.custom_op(f"{_NS}::fwht32", mutates_args=())
def fwht32(x: torch.Tensor) -> torch.Tensor:
    """fwht_block32 (lattice.py:91-102) of every 32-element block along the last dim, one HIP
    kernel, bit-identical to the reference's torch stages (fp32, fp16, bf16, fp64)."""
    dev = N.require_device(x)
    if x.dtype not in _FWHT_CODE:
        raise RuntimeError(f"fwht32 supports float32/float16/bfloat16/float64 (got {x.dtype})")
    if x.shape[-1] == 0 or x.shape[-1] % 32 != 0:
        raise RuntimeError(f"last dimension must be a positive multiple of 32 (got {x.shape[-1]})")
    xc = x.contiguous()
    out = torch.empty_like(xc)
    with torch.cuda.device(dev):
        N.check(N.lib().ojx_fwht32(N.ptr(xc), _FWHT_CODE[x.dtype], xc.numel(), N.ptr(out),
                                   N.stream_handle(dev)),
                "fwht32")
    return out


@fwht32.register_fake
def _(x):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def _fwht32_setup(ctx, inputs, output):
    pass


def _fwht32_backward(ctx, grad):
    # the normalised Hadamard matrix is symmetric: the vector-Jacobian product is the transform
    return fwht32(grad.contiguous())


fwht32.register_autograd(_fwht32_backward, setup_context=_fwht32_setup)


# --------------------------------------------------------------------------- QAT helpers

@torch.library.custom_op(f"{_NS}::cs_project", mutates_args=())
def cs_project(x: torch.Tensor) -> torch.Tensor:
    """Conway-Sloane nearest E8 point of every 8-vector of x (last dim 8) as
    conway_sloane_e8_project's torch path computes it (lattice.py:180-203) in x's dtype:
    float32, float64, or float16 / bfloat16 with every op rounded to that dtype."""
    dev = N.require_device(x)
    if x.dtype not in (torch.float32, torch.float64, torch.float16, torch.bfloat16):
        raise RuntimeError(f"cs_project supports float32, float64, float16 and bfloat16 "
                           f"tensors (got {x.dtype})")
    if x.shape[-1] != 8:
        raise RuntimeError(f"last dimension must be 8 (got {x.shape[-1]})")
    xc = x.contiguous()
    out = torch.empty_like(xc)
    code = N.F64 if x.dtype == torch.float64 else N.DTYPE_CODE[x.dtype]
    with torch.cuda.device(dev):
        N.check(N.lib().ojx_e8_cs_project_dt(N.ptr(xc), code, xc.numel() // 8, N.ptr(out),
                                             N.stream_handle(dev)),
                "e8 cs_project")
    return out


@cs_project.register_fake
def _(x):
    return torch.empty_like(x)


@torch.library.custom_op(f"{_NS}::ste_quantize", mutates_args=())
def ste_quantize(w: torch.Tensor) -> torch.Tensor:
    """Forward of _E8STEFunction (lattice.py:853-865) in w's dtype (float32, float16 or
    bfloat16; the half types round every op as the reference's torch expressions do)."""
    dev = N.require_device(w)
    if w.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"ste_quantize supports float32, float16 and bfloat16 weights "
                           f"(got {w.dtype})")
    wc = w.contiguous()
    out = torch.empty_like(wc)
    with torch.cuda.device(dev):
        N.check(N.lib().ojx_e8_ste_quantize_dt(N.ptr(wc), N.DTYPE_CODE[w.dtype], wc.numel(),
                                               N.ptr(out), N.stream_handle(dev)),
                "e8 ste_quantize")
    return out


@ste_quantize.register_fake
def _(w):
    return torch.empty_like(w)
