"""Pins the 1-bit Root-E8 part of the CPU oracle (oracle/e8t_oracle.c, ojo_e8r_*).

RootE8LatticePacker (ojasx2/math/lattice.py:426-533) is written as torch calls; the
reference ships no golden vectors for it, and its tests check the table's geometry, the
sizes and an SQNR bound (tests/test_tilelang_and_root_e8.py:44-96) and row-wise ==
whole-matrix bytes (tests/test_streaming_e8.py:15-39).  Each check here is independent of
the oracle's C code:
  * table          -> the reference's construction (loops + itertools.product), its
                      geometry test (240 roots of norm^2 8, 16 axes of norm^2 4, E8
                      membership, no duplicates)
  * pack           -> the reference's expression evaluated by torch itself (torch.norm,
                      F.normalize, torch.matmul, torch.argmax, torch.sum), bit for bit
  * sum order      -> torch.sum along a contiguous last dim, every multiple of 8 <= 256
  * argmax rule    -> float64 dot products: the chosen row is within rounding of the
                      best normalised dot
  * MMSE scale     -> <w - s q, q> = 0 for the fp32 scale (the defining property)
  * decode rule    -> torch's own lut.to(dtype)[codes] * scales.to(dtype)
  * dequant-matmul -> float64 matmul of the torch-decoded weights
"""

import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O


def _reference_lut():
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
    return torch.tensor(pts, dtype=torch.float32) * 2.0


def _torch_pack(w, group_size):
    """lattice.py:476-509 as torch calls (the reference's own expression)."""
    if group_size <= 0 or group_size % 8 != 0:
        group_size = 8
    lut = _reference_lut()
    flat = w.reshape(-1).to(torch.float32)
    pad_len = (-flat.numel()) % group_size
    if pad_len > 0:
        flat = F.pad(flat, (0, pad_len))
    w_groups = flat.view(-1, group_size)
    init_scales = torch.norm(w_groups, dim=-1, keepdim=True) / math.sqrt(group_size) + 1e-8
    v = (w_groups / init_scales).view(-1, 8)
    lut_norm = F.normalize(lut, dim=-1)
    dots = torch.matmul(v, lut_norm.t())
    packed = torch.argmax(dots, dim=-1).to(torch.uint8)
    q_groups = lut[packed.to(torch.int32)].view(-1, group_size)
    q_norm_sq = torch.sum(q_groups * q_groups, dim=-1, keepdim=True).clamp(min=1e-8)
    mmse = torch.sum(w_groups * q_groups, dim=-1, keepdim=True) / q_norm_sq
    return packed, mmse.squeeze(-1).to(torch.float16)


def _u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_e8r_table_is_the_reference_table_and_geometry():
    lut = O.e8r_lut()
    assert np.array_equal(lut, _reference_lut().numpy())
    norms = (lut.astype(np.float64) ** 2).sum(-1)
    assert np.all(norms[:240] == 8.0) and np.all(norms[240:] == 4.0)
    assert np.all(lut == np.round(lut)) and np.all(lut.sum(-1) % 2 == 0)
    assert np.unique(lut, axis=0).shape[0] == 256


@pytest.mark.parametrize("gs", [8, 16, 24, 32, 40, 64, 128])
def test_e8r_pack_matches_torch_evaluation_of_reference(gs):
    g = torch.Generator().manual_seed(700 + gs)
    w = torch.randn(96, 256, generator=g) * 0.02
    idx = torch.randperm(w.numel(), generator=g)[:60]
    w.view(-1)[idx] = 0.16 * torch.sign(torch.randn(60, generator=g))  # +-8 sigma outliers
    w[:3] = 0.0  # zero groups: argmax ties at index 0, scale 0
    w[3, :8] = -0.0
    ref_codes, ref_scales = _torch_pack(w, gs)
    codes, s16, _ = O.e8r_encode(w.numpy(), gs)
    assert np.array_equal(codes, ref_codes.numpy())
    assert np.array_equal(s16, _u16(ref_scales))


@pytest.mark.parametrize("shape,gs", [((7, 13), 8), ((5, 19), 16), ((3, 40), 32), ((1, 1), 8),
                                      ((33, 17), 64), ((4, 10), 12)])
def test_e8r_pack_padding_and_coercion(shape, gs):
    g = torch.Generator().manual_seed(sum(shape) + gs)
    w = torch.randn(*shape, generator=g)
    ref_codes, ref_scales = _torch_pack(w, gs)
    codes, s16, _ = O.e8r_encode(w.numpy(), gs)  # gs 12 -> 8, as lattice.py:485-486
    assert np.array_equal(codes, ref_codes.numpy())
    assert np.array_equal(s16, _u16(ref_scales))


def test_e8r_pack_fp16_source_with_ties():
    # fp16 weights repeat values, so exact ties between rows are common: first index wins
    g = torch.Generator().manual_seed(91)
    w = (torch.randint(-3, 4, (64, 128), generator=g).float() * 0.01).half().float()
    ref_codes, ref_scales = _torch_pack(w, 32)
    codes, s16, _ = O.e8r_encode(w.numpy(), 32)
    assert np.array_equal(codes, ref_codes.numpy())
    assert np.array_equal(s16, _u16(ref_scales))


def test_e8r_quantize_matches_torch_argmax_of_matmul():
    g = torch.Generator().manual_seed(5)
    v = torch.randn(200_000, 8, generator=g) * torch.rand(200_000, 1, generator=g) * 4
    lut = _reference_lut()
    ref = torch.argmax(torch.matmul(v, F.normalize(lut, dim=-1).t()), dim=-1)
    assert np.array_equal(O.e8r_quantize8_many(v.numpy()), ref.numpy())


def test_e8r_argmax_is_best_normalised_dot_in_float64():
    rng = np.random.default_rng(3)
    v = rng.standard_normal((20_000, 8)).astype(np.float32)
    codes = O.e8r_quantize8_many(v)
    u = O.e8r_lut().astype(np.float64)
    u /= np.linalg.norm(u, axis=-1, keepdims=True)
    dots = v.astype(np.float64) @ u.T
    chosen = dots[np.arange(v.shape[0]), codes]
    assert np.all(chosen >= dots.max(-1) - 1e-5)


@pytest.mark.parametrize("n", list(range(8, 257, 8)))
def test_e8r_row_sum_is_torch_sum_order(n):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(400, n, generator=g) * torch.rand(400, 1, generator=g) * 10
    ref = x.sum(-1).numpy()
    got = np.array([O.e8r_row_sum(r) for r in x.numpy()], dtype=np.float32)
    assert np.array_equal(got, ref)


def test_e8r_mmse_scale_is_orthogonal_projection():
    g = torch.Generator().manual_seed(11)
    w = torch.randn(32, 64, generator=g)
    codes, _, s32 = O.e8r_encode(w.numpy(), 32)
    lut = O.e8r_lut().astype(np.float64)
    q = lut[codes.astype(np.int64)].reshape(-1, 32)
    wg = w.numpy().astype(np.float64).reshape(-1, 32)
    resid = ((wg - s32[:, None].astype(np.float64) * q) * q).sum(-1)
    assert np.all(np.abs(resid) <= 1e-5 * np.abs(wg * q).sum(-1))


@pytest.mark.parametrize("dtype", [O.DT_F32, O.DT_F16, O.DT_BF16])
def test_e8r_decode_rule_matches_torch(dtype):
    tdt = {O.DT_F32: torch.float32, O.DT_F16: torch.float16, O.DT_BF16: torch.bfloat16}[dtype]
    rng = np.random.default_rng(dtype)
    codes = rng.integers(0, 256, 512, dtype=np.uint8)
    s16 = (rng.standard_normal(128) * 0.05).astype(np.float16)
    s16[:4] = [0.0, -0.0, 6e-8, 40000.0]  # zero, negative zero, subnormal, 2s > fp16 max
    s16b = s16.view(np.uint16)
    lut = _reference_lut().to(tdt)
    ref = (lut[torch.from_numpy(codes.astype(np.int64))].view(-1, 32) *
           torch.from_numpy(s16).to(tdt).view(-1, 1)).reshape(-1)
    got = O.e8r_decode(codes, s16b, 4096, 32, dtype)
    if dtype == O.DT_F32:
        assert np.array_equal(got.view(np.uint32), ref.numpy().view(np.uint32))
    else:
        assert np.array_equal(got, _u16(ref))


def test_e8r_gemm_f64_is_matmul_of_decoded_weights():
    rng = np.random.default_rng(7)
    M, N, K, gs = 3, 40, 96, 16
    w = rng.standard_normal((N, K)).astype(np.float32) * 0.02
    codes, s16, _ = O.e8r_encode(w, gs)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    for dt in (O.DT_F32, O.DT_BF16):
        wd = O.e8r_decode(codes, s16, N * K, gs, dt)
        wd = wd if dt == O.DT_F32 else O.bf16_bits_to_f32(wd)
        ref = x.astype(np.float64) @ wd.reshape(N, K).astype(np.float64).T + bias
        got = O.e8r_gemm_f64(x, codes, s16, bias, N, K, gs, dt)
        assert np.allclose(got, ref, rtol=0, atol=1e-9)
        gy = rng.standard_normal((M, N)).astype(np.float32)
        gx = O.e8r_gemm_bwd_f64(gy, codes, s16, N, K, gs, dt)
        assert np.allclose(gx, gy.astype(np.float64) @ wd.reshape(N, K).astype(np.float64),
                           rtol=0, atol=1e-9)


def test_e8r_reference_invariants():
    # tests/test_tilelang_and_root_e8.py:65-96 of the reference: 1 byte per 8 weights,
    # one scale per group, SQNR above 4 dB on Gaussian weights
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 128, generator=g)
    codes, s16, _ = O.e8r_encode(x.numpy(), 32)
    assert codes.size == 64 * 128 // 8 and s16.size == 64 * 128 // 32
    y = O.e8r_decode(codes, s16, x.numel(), 32, O.DT_F32).reshape(64, 128)
    sqnr = 10 * np.log10((x.numpy() ** 2).mean() / ((x.numpy() - y) ** 2).mean())
    assert sqnr > 4.0
