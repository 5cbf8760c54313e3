"""Pins the Conway-Sloane projection and the QAT straight-through quantizer of the CPU
oracle (oracle/e8t_oracle.c: ojo_e8_cs_project_*, ojo_e8_ste_quantize_f32 and the fp16 /
bf16 forms ojo_e8_cs_project_half, ojo_e8_ste_quantize_half).

The reference's projection (ojasx2/math/lattice.py:180-203) and _E8STEFunction
(:853-865) are torch expressions: each check evaluates them with torch itself, bit for
bit, plus the lattice's defining properties (every output is an E8 point, and it is a
nearest one: no E8 point from a brute-force neighbourhood search is closer in float64)."""

import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O


def cs_torch(x_flat):
    """lattice.py:180-203 (the torch path) verbatim in torch calls."""
    f1 = torch.round(x_flat)
    sum1 = torch.sum(f1, dim=-1, keepdim=True).long()
    err1 = torch.abs(x_flat - f1)
    worst1 = torch.argmax(err1, dim=-1, keepdim=True)
    sign1 = torch.sign(x_flat - f1)
    sign1 = torch.where(sign1 == 0, torch.ones_like(sign1), sign1)
    f1_fixed = f1.scatter(-1, worst1, f1.gather(-1, worst1) + sign1.gather(-1, worst1))
    c1 = torch.where((sum1 % 2 != 0), f1_fixed, f1)
    x_shift = x_flat - 0.5
    f2 = torch.round(x_shift)
    sum2 = torch.sum(f2, dim=-1, keepdim=True).long()
    err2 = torch.abs(x_shift - f2)
    worst2 = torch.argmax(err2, dim=-1, keepdim=True)
    sign2 = torch.sign(x_shift - f2)
    sign2 = torch.where(sign2 == 0, torch.ones_like(sign2), sign2)
    f2_fixed = f2.scatter(-1, worst2, f2.gather(-1, worst2) + sign2.gather(-1, worst2))
    c2 = torch.where((sum2 % 2 != 0), f2_fixed, f2) + 0.5
    d1 = torch.sum((x_flat - c1) ** 2, dim=-1, keepdim=True)
    d2 = torch.sum((x_flat - c2) ** 2, dim=-1, keepdim=True)
    return torch.where(d1 <= d2, c1, c2)


def ste_torch(w):
    """lattice.py:855-865 verbatim."""
    total = w.numel()
    pad_len = (-total) % 8
    flat = F.pad(w.reshape(-1), (0, pad_len)) if pad_len > 0 else w.reshape(-1)
    w_flat = flat.view(-1, 8)
    scales = torch.norm(w_flat, dim=-1, keepdim=True) / math.sqrt(8) + 1e-8
    w_e8 = cs_torch(w_flat / scales)
    return (w_e8 * scales).reshape(-1)[:total].view(w.shape)


def _inputs(dtype, n=200_000, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, 8, generator=g) * 3).to(dtype)
    x[:2000] = torch.round(x[:2000] * 2) / 2           # exact halves: rounding ties
    x[2000:3000] = torch.round(x[2000:3000])           # lattice-adjacent integers
    x[3000:3100] = 0.0
    x[3100:3200] = -0.0
    x[3200:3300, :] = 0.5                               # equal errors everywhere
    return x


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_cs_project_matches_torch_path(dtype):
    x = _inputs(dtype)
    got = O.cs_project(x.numpy())
    ref = cs_torch(x).numpy()
    assert got.dtype == ref.dtype and np.array_equal(got, ref)


_OFFSETS = np.array(list(itertools.product((-1.0, 0.0, 1.0), repeat=8)))


def test_cs_project_outputs_nearest_e8_point():
    # every output is an E8 point (all integers or all half-integers, even sum) and no E8
    # point within one step per coordinate of either rounding of v is closer (float64)
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((200, 8)) * 2).astype(np.float64)
    out = O.cs_project(x)
    for v, c in zip(x, out):
        assert np.all(c == np.round(c)) or np.all(c - 0.5 == np.round(c - 0.5))
        assert int(round(c.sum())) % 2 == 0
        best = ((v - c) ** 2).sum()
        for base in (np.round(v), np.floor(v) + 0.5):
            pts = base + _OFFSETS
            pts = pts[np.round(pts.sum(-1)).astype(np.int64) % 2 == 0]
            assert best <= ((v - pts) ** 2).sum(-1).min() + 1e-12


def test_ste_quantize_matches_torch_expression():
    g = torch.Generator().manual_seed(4)
    for shape in ((1000, 37), (64, 64), (3, 5), (1, 1)):
        w = torch.randn(*shape, generator=g) * 0.05
        w.view(-1)[: min(4, w.numel())] = 0.0
        assert np.array_equal(O.ste_quantize(w.numpy()), ste_torch(w).numpy())


def _half_inputs(dtype, n=200_000, seed=5):
    x = _inputs(torch.float32, n, seed)
    g = torch.Generator().manual_seed(seed + 1)
    # large magnitudes, where x - 0.5, f +- 1 and the rounded parity sum lose precision in
    # the half type (fp16 integers are exact to 2048, bf16 ones to 256)
    x[4000:6000] = torch.randn(2000, 8, generator=g) * 400
    x[6000:7000] = torch.round(torch.randn(1000, 8, generator=g) * 300)
    x[7000:7100] = torch.tensor([256.0, 1, 1, 1, 1, 1, 1, 1])
    x[7100:7200] = torch.tensor([2048.0, 1, 1, 1, 1, 1, 1, 0.5])
    x[7200:7300] = torch.tensor([1000.5, -3.5, 2.5, 0.5, -0.5, 7.5, 1.5, 0.25])
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_cs_project_half_matches_torch_path(dtype):
    # the reference's torch path evaluated by torch on an fp16 / bf16 tensor: every op
    # rounds to the tensor's dtype (lattice.py:180-203)
    x = _half_inputs(dtype)
    got = O.cs_project_half(x.float().numpy(), dtype == torch.bfloat16)
    ref = cs_torch(x).float().numpy()
    assert np.array_equal(got, ref, equal_nan=True)
    # the half rounding matters: the fp32 projection of the same values differs somewhere
    assert not np.array_equal(O.cs_project(x.float().numpy()), ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_ste_quantize_half_matches_torch_expression(dtype):
    g = torch.Generator().manual_seed(6)
    for shape in ((1000, 37), (64, 64), (3, 5), (1, 1), (256, 256)):
        w = (torch.randn(*shape, generator=g) * 0.05).to(dtype)
        w.view(-1)[: min(4, w.numel())] = 0.0
        if w.numel() >= 64:
            w.view(-1)[8:16] = 0.0          # a zero 8-vector: s = rnd(0 + 1e-8) (0 in fp16)
            w.view(-1)[16:24] = 3e-5        # a tiny one
            w.view(-1)[24:32] = torch.tensor([60.0, 1e-3, 0, 0, 0, 0, 0, -2.0])
        got = O.ste_quantize_half(w.float().numpy(), dtype == torch.bfloat16)
        ref = ste_torch(w).float().numpy()
        assert np.array_equal(got, ref, equal_nan=True), shape
