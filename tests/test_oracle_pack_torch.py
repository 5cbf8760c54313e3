"""Pins the ternary and 2-bit encoders of the CPU oracle as whole pipelines.

The reference's packers are torch expressions (TernaryE8LatticePacker.pack,
ojasx2/math/lattice.py:338-384; E8LatticePacker.pack, lattice.py:213-249).  Here torch
itself evaluates that arithmetic -- group norms by torch.norm, round-half-even by
torch.round, the parity fix by argmin over the penalty, the code and byte packing -- and
the oracle's C encoder (oracle/e8t_oracle.c) must produce the same bytes and fp16 scale
bits.  The inputs are the configs[0] layer of the benchmark (4096 x 4096 fp32 N(0, 0.02),
seed 8101), a configs[3]-style fp16 layer with 0.1% +-8 sigma outliers, zero groups, and
ragged shapes that need padding and group-size coercion.  The oracle's code is not used
to form the expected values.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O


def _groups(w: torch.Tensor, gs: int):
    flat = w.reshape(-1).to(torch.float32)
    flat = F.pad(flat, (0, (-flat.numel()) % gs))
    g = flat.view(-1, gs)
    s = torch.norm(g, dim=-1, keepdim=True) / math.sqrt(gs) + 1e-8
    return g, s


def _even_fix(q: torch.Tensor, alt: torch.Tensor, target: torch.Tensor, odd: torch.Tensor):
    """Where `odd`, swap in `alt` at the coordinate whose swap costs the least squared error
    (first such coordinate on ties, as torch.argmin)."""
    cost = (alt - target) ** 2 - (q - target) ** 2
    j = cost.argmin(dim=-1, keepdim=True)
    swapped = q.scatter(-1, j, alt.gather(-1, j))
    return torch.where(odd, swapped, q)


def torch_ternary_pack(w: torch.Tensor, gs: int = 32):
    """Ternary-E8 codes (2 per 3 bytes) and fp16 scales, lattice.py:338-384."""
    if gs <= 0 or gs % 16 != 0:
        gs = 16  # lattice.py:346-347
    g, s = _groups(w, gs)
    v = (g / s).view(-1, 8)
    q = torch.round(v).clamp(-1.0, 1.0)
    odd = (q.sum(dim=-1, keepdim=True).long() % 2) != 0
    alt = torch.where(q == 0.0, torch.where(v >= 0.0, 1.0, -1.0), 0.0)
    q = _even_fix(q, alt, v, odd)
    raw = ((q.long() + 1) * (3 ** torch.arange(8))).sum(dim=-1)
    code = raw // 2  # rank among the even-parity raw indices (raw is even here)
    assert bool((raw % 2 == 0).all())
    c0, c1 = code.view(-1, 2).unbind(-1)
    packed = torch.stack([c0 & 0xFF, ((c0 >> 8) & 0x0F) | ((c1 & 0x0F) << 4), (c1 >> 4) & 0xFF],
                         dim=-1).to(torch.uint8).flatten()
    return packed, s.squeeze(-1).to(torch.float16)


def torch_e8b_pack(w: torch.Tensor, gs: int = 8):
    """2-bit E8 codes (4 per byte) and fp16 scales, lattice.py:213-249."""
    g, s = _groups(w, gs)
    t = (g / s).view(-1, 8) - 0.5
    f = torch.round(t).clamp(-2.0, 1.0)
    odd = (f.sum(dim=-1, keepdim=True).long() % 2) != 0
    alt = torch.where(t >= f, (f + 1.0).clamp(-2.0, 1.0), (f - 1.0).clamp(-2.0, 1.0))
    f = _even_fix(f, alt, t, odd)
    codes = torch.round(f + 0.5 + 1.5).clamp(0, 3).to(torch.uint8).view(-1, 4)
    packed = codes[:, 0] | (codes[:, 1] << 2) | (codes[:, 2] << 4) | (codes[:, 3] << 6)
    return packed, s.squeeze(-1).to(torch.float16)


def _u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _c1_layer():
    return torch.randn(4096, 4096, generator=torch.Generator().manual_seed(8101)) * 0.02


def _outlier_layer(rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(rows, cols, generator=g) * 0.02).to(torch.float16)
    n = max(1, w.numel() // 1000)
    idx = torch.randperm(w.numel(), generator=g)[:n]
    w.view(-1)[idx] = (0.16 * torch.sign(torch.randn(n, generator=g))).to(torch.float16)
    return w


def _check_ternary(w, gs):
    ref_p, ref_s = torch_ternary_pack(w, gs)
    p, s16, _ = O.encode(w.float().numpy(), gs)
    assert np.array_equal(p, ref_p.numpy())
    assert np.array_equal(s16, _u16(ref_s))


def _check_e8b(w, gs):
    ref_p, ref_s = torch_e8b_pack(w, gs)
    p, s16, _ = O.e8b_encode(w.float().numpy(), gs)
    assert np.array_equal(p, ref_p.numpy())
    assert np.array_equal(s16, _u16(ref_s))


def test_ternary_oracle_equals_torch_pack_on_c1_layer():
    _check_ternary(_c1_layer(), 32)


def test_e8b_oracle_equals_torch_pack_on_c1_layer():
    _check_e8b(_c1_layer(), 8)
    _check_e8b(_c1_layer()[:1024], 32)


@pytest.mark.parametrize("gs", [16, 32, 64])
def test_ternary_oracle_equals_torch_pack_with_outliers(gs):
    w = _outlier_layer(512, 1024, 9000 + gs)
    w[:2] = 0.0   # zero groups: scale 1e-8, all-zero codes
    w[2, :16] = -0.0
    _check_ternary(w, gs)


@pytest.mark.parametrize("gs", [8, 16, 32])
def test_e8b_oracle_equals_torch_pack_with_outliers(gs):
    w = _outlier_layer(512, 1024, 9100 + gs)
    w[:2] = 0.0
    _check_e8b(w, gs)


@pytest.mark.parametrize("shape,gs", [((7, 13), 32), ((5, 19), 16), ((3, 40), 24), ((1, 1), 32),
                                      ((33, 17), 64), ((4, 10), 0)])
def test_ternary_oracle_equals_torch_pack_padding_and_coercion(shape, gs):
    w = torch.randn(*shape, generator=torch.Generator().manual_seed(sum(shape) + gs))
    _check_ternary(w, gs)


@pytest.mark.parametrize("shape,gs", [((7, 13), 8), ((5, 19), 16), ((3, 40), 24), ((1, 1), 8),
                                      ((33, 17), 64)])
def test_e8b_oracle_equals_torch_pack_padding(shape, gs):
    w = torch.randn(*shape, generator=torch.Generator().manual_seed(sum(shape) + gs + 1))
    _check_e8b(w, gs)


def test_pack_round_half_even_ties():
    # coordinates exactly at +-0.5 / +-1.5 after normalisation: torch.round takes the even
    # neighbour; both pipelines must agree.  A group of eight equal magnitudes has scale
    # |a| (+1e-8), so v = +-1 exactly; halves come from mixing a and a/2 with the right norm.
    rows = []
    for signs in range(16):
        r = np.array([1.0 if (signs >> i) & 1 else -1.0 for i in range(4)] * 8, np.float32)
        rows.append(r * 0.03)
        r2 = r.copy()
        r2[::2] *= 0.5
        rows.append(r2 * 0.03)
    w = torch.from_numpy(np.stack(rows))
    _check_ternary(w, 32)
    _check_e8b(w, 8)
    _check_e8b(w, 32)
