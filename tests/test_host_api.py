"""Host-side checks that need no GPU: the C ABI library loads and exports every
declared symbol, argument validation rejects bad calls before any launch, and
the Python layer keeps the reference's shapes, coercions and errors."""

import ctypes
import math
import os
import re

import numpy as np
import pytest
import torch
import torch.nn as nn

import ojasx_amd
from ojasx_amd import _native as N
from ojasx_amd import lattice as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ojasx_e8t.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(ojx_\w+)\s*\(", text)))


def test_header_declares_the_exports():
    assert _declared_symbols() == sorted(N.EXPORTS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = N.lib()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    assert lib.ojx_e8t_version() >= 20000


def test_library_has_gfx950_code_object():
    # the HIP fat binary embeds the target id; the library must carry gfx950 code
    with open(N.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"gfx950" in blob


def test_abi_rejects_bad_arguments_before_launch():
    lib = N.lib()
    # negative sizes, unknown dtype and bad group size fail without touching a GPU
    assert lib.ojx_e8t_encode(None, 0, -1, 32, None, None, None) == -1
    assert lib.ojx_e8t_encode(None, 7, 16, 32, None, None, None) == -3
    assert lib.ojx_e8t_encode(None, 0, 16, 24, None, None, None) == -2
    assert b"multiple of 16" in lib.ojx_e8t_last_error()
    assert lib.ojx_e8t_decode(None, None, 16, 0, 0, None, None) == -2
    assert lib.ojx_e8t_gemm_fwd(None, None, None, None, None, -1, 4, 4, 32, 0, None, 0, None) == -1
    assert lib.ojx_e8t_gemm_fwd(None, None, None, None, None, 1, 4, 4, 32, 9, None, 0, None) == -3
    assert lib.ojx_e8t_gemm_fwd(None, None, None, None, None, 1, 4, 32, 32, 0, None, 0, None) == -1
    assert lib.ojx_e8t_gemm_bwd_dx(None, None, None, None, 1, 4, 32, 20, 2, None, 0, None) == -2
    # empty work is a no-op success
    assert lib.ojx_e8t_encode(None, 0, 0, 32, None, None, None) == 0
    assert lib.ojx_e8t_gemm_fwd(None, None, None, None, None, 0, 4, 4, 32, 0, None, 0, None) == 0
    # 2-bit: the packer's group rule (multiple of 8), the native op's (multiple of 4)
    assert lib.ojx_e8_encode(None, 0, 64, 12, None, None, None) == -2
    assert b"multiple of 8" in lib.ojx_e8t_last_error()
    assert lib.ojx_e8_encode(None, 0, -1, 8, None, None, None) == -1
    assert lib.ojx_e8_decode(None, None, 16, 4, 0, None, None) == -2
    assert lib.ojx_e8_gemm_fwd(None, None, None, None, None, 1, 4, 8, 6, 0, None, 0, None) == -2
    assert b"multiple of 4" in lib.ojx_e8t_last_error()
    assert lib.ojx_e8_gemm_fwd(None, None, None, None, None, 1, 4, 8, 4, 9, None, 0, None) == -3
    assert lib.ojx_e8_gemm_bwd_dx(None, None, None, None, -1, 4, 8, 8, 0, None, 0, None) == -1
    assert lib.ojx_e8_encode(None, 0, 0, 8, None, None, None) == 0
    assert lib.ojx_e8_gemm_fwd(None, None, None, None, None, 0, 4, 8, 8, 0, None, 0, None) == 0
    # 1-bit Root E8: group sizes are multiples of 8 everywhere (the packer coerces first)
    assert lib.ojx_e8r_encode(None, 0, 64, 12, None, None, None) == -2
    assert b"multiple of 8" in lib.ojx_e8t_last_error()
    assert lib.ojx_e8r_encode(None, 0, -1, 8, None, None, None) == -1
    assert lib.ojx_e8r_decode(None, None, 16, 4, 0, None, None) == -2
    assert lib.ojx_e8r_gemm_fwd(None, None, None, None, None, 1, 4, 8, 4, 0, None, 0, None) == -2
    assert lib.ojx_e8r_gemm_fwd(None, None, None, None, None, 1, 4, 8, 8, 9, None, 0, None) == -3
    assert lib.ojx_e8r_gemm_bwd_dx(None, None, None, None, -1, 4, 8, 8, 0, None, 0, None) == -1
    assert lib.ojx_e8r_encode(None, 0, 0, 8, None, None, None) == 0
    # a workspace size without a workspace, or a misaligned one, is refused before any launch
    assert lib.ojx_e8t_gemm_fwd(None, None, None, None, None, 0, 4, 4, 32, 0, None, 64,
                                None) == -1
    assert lib.ojx_e8t_gemm_fwd(None, None, None, None, None, 0, 4, 4, 32, 0, 8, 64, None) == -2
    assert lib.ojx_e8r_gemm_fwd(None, None, None, None, None, 0, 4, 8, 8, 0, None, 0, None) == 0
    # the LoRA forward checks every operand, the workspace included, before it enqueues the
    # down-projection (fake but aligned device addresses; nothing here reaches a GPU call)
    A, X, P, S, Y, U, B = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 0x60000, 0x70000
    for f in (lib.ojx_e8t_gemm_fwd_lora, lib.ojx_e8_gemm_fwd_lora, lib.ojx_e8r_gemm_fwd_lora):
        args = dict(x=X, p=P, s=S, bias=None, a=A, b=B, r=8, sc=2.0, u=U, y=Y, M=1, N=64, K=256,
                    gs=32, dt=2, ws=None, wsb=0)

        def call(**kw):
            a = dict(args, **kw)
            return f(a["x"], a["p"], a["s"], a["bias"], a["a"], a["b"], a["r"], a["sc"], a["u"],
                     a["y"], a["M"], a["N"], a["K"], a["gs"], a["dt"], a["ws"], a["wsb"], None)

        assert call(u=U + 2) == -2 and b"misaligned LoRA" in lib.ojx_e8t_last_error()
        assert call(b=B + 1) == -2
        assert call(a=A + 1) == -2
        assert call(wsb=64) == -1 and b"null workspace" in lib.ojx_e8t_last_error()
        assert call(ws=0x80008, wsb=64) == -2
        assert call(r=0) == -2 and call(r=65) == -2
        assert call(u=None) == -1
        assert call(M=0) == 0


def test_ops_refuse_cpu_tensors():
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        ojasx_amd.ops.encode(torch.randn(4, 32), 32)
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        ojasx_amd.ops.e8t_linear(torch.randn(2, 32), torch.zeros(6, dtype=torch.uint8),
                                 torch.ones(2, dtype=torch.float16), None, 2, 32, 32)


@pytest.mark.parametrize("gs,eff", [(8, 16), (24, 16), (16, 16), (32, 32), (64, 64)])
def test_layer_buffer_shapes_and_group_coercion(gs, eff):
    # lattice.py:748-767 (bitrate 1.5 branch)
    layer = ojasx_amd.E8LatticeLinear(128, 96, rank=4, group_size=gs, bitrate=1.5)
    assert layer.group_size == eff
    total = 128 * 96
    padded = total + ((-total) % eff)
    assert layer.packed_weight.shape == (padded * 3 // 16,)
    assert layer.packed_weight.dtype == torch.uint8
    assert layer.block_scales.shape == (padded // eff,)
    assert layer.block_scales.dtype == torch.float16
    assert layer.lora_A.shape == (128, 4) and layer.lora_B.shape == (4, 96)
    assert layer.scaling == 16.0 / 4


def test_layer_state_dict_keys_match_reference():
    layer = ojasx_amd.E8LatticeLinear(64, 32, bias=True, rank=2, group_size=32, bitrate=1.5)
    assert set(layer.state_dict()) == {"packed_weight", "block_scales", "bias", "lora_A", "lora_B"}


def test_bitrate_routing():
    # lattice.py:536-541: 1.0 -> RootE8LatticePacker, 1.5 -> ternary, anything else -> 2-bit
    assert ojasx_amd._get_packer_for_bitrate(1.0) is ojasx_amd.RootE8LatticePacker
    assert ojasx_amd._get_packer_for_bitrate(2.0) is ojasx_amd.E8LatticePacker
    assert ojasx_amd._get_packer_for_bitrate(3.0) is ojasx_amd.E8LatticePacker
    assert ojasx_amd._get_packer_for_bitrate(1.5) is ojasx_amd.TernaryE8LatticePacker


@pytest.mark.parametrize("gs,eff", [(8, 8), (4, 8), (12, 8), (16, 16), (32, 32), (40, 40)])
def test_1bit_layer_buffer_shapes_and_group_coercion(gs, eff):
    # lattice.py:756-767 (1.0 branch): group >= 8 and a multiple of 8, else 8; 1 byte / 8
    layer = ojasx_amd.E8LatticeLinear(128, 96, rank=2, group_size=gs, bitrate=1.0)
    assert layer.group_size == eff
    total = 128 * 96
    padded = total + ((-total) % eff)
    assert layer.packed_weight.shape == (padded // 8,)
    assert layer.block_scales.shape == (padded // eff,)


def test_root_e8_lut_matches_reference_construction():
    # the table as lattice.py:436-456 builds it (loops and itertools.product), scaled by 2
    import itertools
    pts = []
    for i in range(8):
        for j in range(i + 1, 8):
            for s1 in (-1.0, 1.0):
                for s2 in (-1.0, 1.0):
                    vec = [0.0] * 8
                    vec[i], vec[j] = s1, s2
                    pts.append(vec)
    for signs in itertools.product((-0.5, 0.5), repeat=8):
        if sum(1 for s in signs if s < 0) % 2 == 0:
            pts.append(list(signs))
    for i in range(8):
        for s in (-1.0, 1.0):
            vec = [0.0] * 8
            vec[i] = s
            pts.append(vec)
    ref = torch.tensor(pts, dtype=torch.float32) * 2.0
    assert torch.equal(ojasx_amd._get_root_e8_lut(), ref)


@pytest.mark.parametrize("gs,eff", [(8, 8), (4, 8), (12, 8), (16, 16), (32, 32), (24, 24)])
def test_2bit_layer_buffer_shapes_and_group_coercion(gs, eff):
    # lattice.py:756-767 (2-bit branch): group >= 8 and a multiple of 8, else 8
    layer = ojasx_amd.E8LatticeLinear(128, 96, rank=2, group_size=gs, bitrate=2.0)
    assert layer.group_size == eff
    total = 128 * 96
    padded = total + ((-total) % eff)
    assert layer.packed_weight.shape == (padded // 4,)
    assert layer.block_scales.shape == (padded // eff,)


def test_2bit_packer_group_size_error():
    # lattice.py:220-221: ValueError, not a coercion
    with pytest.raises(ValueError, match="multiple of 8"):
        ojasx_amd.E8LatticePacker.pack(torch.randn(4, 32), group_size=12)


def test_rowwise_layout_validation_messages():
    # streaming_e8.py:90-109 (reference tests/test_streaming_e8.py:42-47)
    with pytest.raises(ValueError, match="not divisible"):
        ojasx_amd.pack_weight_rowwise(torch.randn(2, 30), group_size=32)
    with pytest.raises(ValueError, match="multiple of 32"):
        ojasx_amd.pack_weight_rowwise(torch.randn(2, 48), group_size=24)
    with pytest.raises(ValueError, match="rank-2"):
        ojasx_amd.pack_weight_rowwise(torch.randn(2, 4, 32))


def test_ternary_luts_closed_form():
    r2c, raw2rank, powers = ojasx_amd._get_ternary_e8_luts()
    assert r2c.shape == (3281, 8) and r2c.dtype == torch.int8
    raw = ((r2c.long() + 1) * powers).sum(dim=1)
    assert torch.equal(raw, 2 * torch.arange(3281))
    assert torch.equal(raw2rank[raw], torch.arange(3281))


def test_fwht_block32_is_normalised_hadamard_and_involution():
    from scipy.linalg import hadamard

    x = torch.randn(7, 96, dtype=torch.float64)
    H = torch.from_numpy(hadamard(32).astype(np.float64)) / math.sqrt(32)
    ref = (x.view(7, 3, 32) @ H.T).view(7, 96)
    assert torch.allclose(L.fwht_block32(x), ref, atol=1e-12)
    assert torch.allclose(L.fwht_block32(L.fwht_block32(x)), x, atol=1e-12)
    y = torch.randn(3, 30)
    assert L.fwht_block32(y) is y  # not a multiple of 32: unchanged


def test_fwht_block32_matches_stagewise_butterflies_bitwise():
    # lattice.py:95-101 combines pairs at distance 1, then 2, 4, 8, 16 with the sum
    # in the lower slot; the same rounded ops in another order change low bits.
    x = torch.randn(64, 32)
    h = x.clone()
    for d in (1, 2, 4, 8, 16):
        out = h.clone()
        for i in range(32):
            if (i // d) % 2 == 0:
                out[:, i] = h[:, i] + h[:, i + d]
                out[:, i + d] = h[:, i] - h[:, i + d]
        h = out
    ref = h * 0.1767766952966369
    assert torch.equal(L.fwht_block32(x), ref)


def test_ctypes_signatures_match_header_arity():
    text = open(HEADER).read()
    lib = N.lib()
    for name in N.EXPORTS:
        m = re.search(name + r"\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(getattr(lib, name).argtypes) == len(params), name


def test_checkpoint_loader_argument_errors(tmp_path):
    # streaming_e8.py:286-298: argument checks come before any file or device access
    with pytest.raises(ValueError, match="row_block must be positive"):
        ojasx_amd.load_hf_checkpoint_e8(str(tmp_path), row_block=0)
    with pytest.raises(ValueError, match="lora_rank must be non-negative"):
        ojasx_amd.load_hf_checkpoint_e8(str(tmp_path), lora_rank=-1)
    with pytest.raises(ValueError, match="Unsupported E8 bitrate"):
        ojasx_amd.load_hf_checkpoint_e8(str(tmp_path), bitrate=3.0)
    with pytest.raises(ValueError, match="multiple of 32"):
        ojasx_amd.load_hf_checkpoint_e8(str(tmp_path), group_size=48)
    with pytest.raises(NotADirectoryError):
        ojasx_amd.load_hf_checkpoint_e8(str(tmp_path / "absent"))


def _fwht_stagewise(x):
    # the reference's loop (lattice.py:112-122): in-place halves at distance h, then / sqrt(n)
    n = x.shape[-1]
    out = x.clone()
    h = 1
    while h < n:
        out = out.view(-1, n // (2 * h), 2, h)
        a = out[:, :, 0, :].clone()
        b = out[:, :, 1, :].clone()
        out[:, :, 0, :] = a + b
        out[:, :, 1, :] = a - b
        h *= 2
    return out.view(x.shape) / math.sqrt(n)


@pytest.mark.parametrize("n", [1, 2, 8, 64, 256, 1024])
def test_fast_walsh_hadamard_transform_bitwise_and_orthonormal(n):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(3, 5, n, generator=g)
    y = ojasx_amd.fast_walsh_hadamard_transform(x)
    assert torch.equal(y, _fwht_stagewise(x))
    assert torch.allclose(ojasx_amd.fast_walsh_hadamard_transform(y), x, atol=1e-5)
    assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), rtol=1e-5)
    with pytest.raises(ValueError, match="power of 2"):
        ojasx_amd.fast_walsh_hadamard_transform(torch.zeros(2, 12))
    assert torch.equal(ojasx_amd.fast_walsh_hadamard_transform(x[..., :32] if n >= 32 else
                                                                torch.zeros(1, 32)),
                       ojasx_amd.fwht_block32(x[..., :32] if n >= 32 else torch.zeros(1, 32)))


def test_randomized_hadamard_transform_matches_reference_steps():
    w = torch.randn(64, 128, generator=torch.Generator().manual_seed(1))
    rot, s1, s2 = ojasx_amd.randomized_hadamard_transform(w, seed=42)
    rng = torch.Generator().manual_seed(42)
    e1 = torch.randint(0, 2, (64,), generator=rng, dtype=w.dtype) * 2 - 1
    e2 = torch.randint(0, 2, (128,), generator=rng, dtype=w.dtype) * 2 - 1
    assert torch.equal(s1, e1) and torch.equal(s2, e2)
    signed = (w * e2.unsqueeze(0)) * e1.unsqueeze(1)
    ref = _fwht_stagewise(_fwht_stagewise(signed).transpose(0, 1)).transpose(0, 1)
    assert torch.equal(rot, ref)
    # non-power-of-two rows with a multiple-of-32 width: fwht_block32 along rows
    w2 = torch.randn(48, 96, generator=torch.Generator().manual_seed(2))
    rot2, a1, a2 = ojasx_amd.randomized_hadamard_transform(w2, seed=7)
    assert torch.equal(rot2, ojasx_amd.fwht_block32((w2 * a2.unsqueeze(0)) * a1.unsqueeze(1)))
    # neither: signs only
    w3 = torch.randn(5, 7)
    rot3, b1, b2 = ojasx_amd.randomized_hadamard_transform(w3, seed=None)
    assert torch.equal(rot3, (w3 * b2.unsqueeze(0)) * b1.unsqueeze(1))


def _ws(fmt, bwd, M, N_out, K, gs=32, dtype=N.BF16):
    n = ctypes.c_size_t(123)
    st = N.lib().ojx_gemm_workspace_bytes(fmt, bwd, M, N_out, K, gs, dtype, ctypes.byref(n))
    assert st == 0, N.lib().ojx_e8t_last_error()
    return n.value


def test_workspace_query_follows_the_dispatch():
    """ojx_gemm_workspace_bytes is host-only logic: decode GEMVs and large prefill grids need
    no scratch; small prefill grids split over K and need splits x M x N fp32 partials."""
    # decode (M <= 16) never needs a workspace, for any format
    for fmt in (0, 1, 2):
        for M in (1, 4, 16):
            assert _ws(fmt, 0, M, 4096, 4096) == 0
    # M = 8192 on a q-shaped layer fills the GPU unsplit
    assert _ws(0, 0, 8192, 4096, 4096) == 0
    # M = 512 on the k/v shape splits: a whole number of M x N fp32 slabs
    b = _ws(0, 0, 512, 1024, 4096)
    assert b > 0 and b % (512 * 1024 * 4) == 0 and b // (512 * 1024 * 4) >= 2
    # backward dX of a small grid also splits (its output is [M, K]) when its reduction (N)
    # has at least 32 steps of 64; the k/v shape's 16 steps at M = 512 run unsplit
    b = _ws(0, 1, 512, 4096, 4096)
    assert b > 0 and b % (512 * 4096 * 4) == 0
    assert _ws(0, 1, 512, 1024, 4096) == 0
    # fp32 activations run the general kernel: no scratch
    assert _ws(0, 0, 512, 1024, 4096, dtype=N.F32) == 0
    # errors: unknown format, bad group size, null result pointer
    n = ctypes.c_size_t(0)
    assert N.lib().ojx_gemm_workspace_bytes(7, 0, 1, 1, 32, 32, 2, ctypes.byref(n)) == -1
    assert N.lib().ojx_gemm_workspace_bytes(0, 0, 1, 1, 32, 24, 2, ctypes.byref(n)) == -2
    assert N.lib().ojx_gemm_workspace_bytes(0, 0, 1, 1, 32, 32, 2, None) == -1
