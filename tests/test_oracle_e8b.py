"""Pins the 2-bit E8 part of the CPU oracle (oracle/e8t_oracle.c, ojo_e8b_*).

The reference (E8LatticePacker, ojasx2/math/lattice.py:209-279) ships no golden
vectors; its own tests check sizes and a cosine bound (tests/test_e8_lattice.py:84-107)
and row-wise == whole-matrix bytes (tests/test_streaming_e8.py:15-39).  Each check
here is independent of the oracle's formulas:
  * group scale        -> torch.norm(...) / math.sqrt(gs) + 1e-8 evaluated by torch
                          (lattice.py:227), group sizes that are multiples of 8
  * nearest-point rule -> exhaustive search over the 32,768 even-parity points of
                          {-1.5, -0.5, 0.5, 1.5}^8 in float64 for vectors that no clamp
                          touches, and hand-derived clamp / tie cases
                          (tests/golden/known_answers_e8b.json)
  * byte layout        -> closed form (c0 | c1<<2 | c2<<4 | c3<<6, lattice.py:242-247)
  * decode rule        -> torch's own (codes.to(dtype) - 1.5) * scales.to(dtype)
                          (lattice.py:274-276)
  * dequant-matmul     -> the reference's C++ 2-bit fused forward / backward
                          (ojasx_math_core.hpp:440-534, via oracle/_ref), tolerance of
                          the reference's fused-GEMM test (abs 1e-4)
"""

import itertools
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("gs", [8, 16, 24, 32, 64])
def test_e8b_group_scale_matches_torch_norm_expression(gs):
    g = torch.Generator().manual_seed(300 + gs)
    w = torch.randn(20000, gs, generator=g) * 0.02
    idx = torch.randperm(w.numel(), generator=g)[: w.numel() // 1000]
    w.view(-1)[idx] = 0.16 * torch.sign(torch.randn(idx.numel(), generator=g))
    w[:50] = 0.0
    ref = (torch.norm(w, dim=-1) / math.sqrt(gs) + 1e-8).numpy()
    _, s16, s32 = O.e8b_encode(w.numpy(), gs)
    assert np.array_equal(_bits(s32), _bits(ref))
    ref16 = torch.from_numpy(ref).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(s16, ref16)


def test_e8b_known_answers():
    with open(os.path.join(GOLDEN, "known_answers_e8b.json")) as f:
        d = json.load(f)
    for c in d["vectors"]:
        got = O.e8b_quantize8_many(np.array(c["v"], dtype=np.float32)).reshape(-1).tolist()
        assert got == c["codes"], c["why"]
    for g in d["groups"]:
        packed, s16, _ = O.e8b_encode(np.array(g["w"], dtype=np.float32), g["gs"])
        assert packed.tolist() == g["bytes"], g["why"]
        assert int(s16[0]) == g["scale16"], g["why"]


_POINTS = None


def _even_points():
    global _POINTS
    if _POINTS is None:
        f = np.array(list(itertools.product([-2, -1, 0, 1], repeat=8)), dtype=np.int64)
        f = f[f.sum(axis=1) % 2 == 0]
        _POINTS = f
    return _POINTS


def test_e8b_rule_is_nearest_even_point_when_unclamped():
    # v in [-1.5, 1.5): xs = v - 0.5 in [-2, 1), so no coordinate is clamped and the
    # rule must return the nearest point of {f + 0.5 : f in {-2..1}^8, sum f even}
    pts = _even_points()
    centers = pts.astype(np.float64) + 0.5
    rng = np.random.default_rng(11)
    v = rng.uniform(-1.5, 1.4999, size=(1500, 8)).astype(np.float32)
    codes = O.e8b_quantize8_many(v).astype(np.int64) - 2  # f2
    checked = 0
    for i in range(0, v.shape[0], 100):
        vb = v[i:i + 100].astype(np.float64)
        d = ((vb[:, None, :] - centers[None, :, :]) ** 2).sum(axis=2)
        order = np.argsort(d, axis=1)
        best, second = order[:, 0], order[:, 1]
        gap = d[np.arange(len(vb)), second] - d[np.arange(len(vb)), best]
        for j in range(len(vb)):
            if gap[j] < 1e-6:
                continue  # a tie: settled by the hand-derived cases
            assert np.array_equal(codes[i + j], pts[best[j]]), (v[i + j], codes[i + j])
            checked += 1
    assert checked > 1400


def test_e8b_clamped_vectors_keep_the_reference_quirk():
    # with a clamped coordinate first among the minimum penalties, the reference leaves an
    # odd sum: the result then differs from the nearest even point by construction
    v = np.array([[1.6] + [0.5] * 7, [-3.0, 1.6] + [0.5] * 6], dtype=np.float32)
    f2 = O.e8b_quantize8_many(v).astype(np.int64) - 2
    assert (f2.sum(axis=1) % 2 == 1).all()


def test_e8b_sizes_and_reference_invariants():
    # tests/test_e8_lattice.py:84-107 of the reference: 64x128, default group size 8
    torch.manual_seed(42)
    w = torch.randn(64, 128) * 0.05
    packed, s16, _ = O.e8b_encode(w.numpy(), 8)
    assert packed.size == w.numel() // 4 and s16.size == w.numel() // 8
    wr = torch.from_numpy(O.e8b_decode(packed, s16, w.numel(), 8)).view(64, 128)
    cos = torch.sum(w * wr) / (torch.norm(w) * torch.norm(wr))
    assert cos.item() > 0.90


def test_e8b_group_size_must_be_multiple_of_8():
    for gs in (0, -8, 12, 20):
        with pytest.raises(ValueError, match="multiple of 8"):
            O.e8b_encode(np.zeros(64, dtype=np.float32), gs)


def test_e8b_byte_layout_closed_form():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal(8 * 64) * 0.02).astype(np.float32)
    packed, s16, s32 = O.e8b_encode(w, 8)
    v = (w.reshape(-1, 8) / s32[:, None]).astype(np.float32)
    codes = O.e8b_quantize8_many(v).reshape(-1)
    c = codes.reshape(-1, 4).astype(np.uint32)
    want = c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)
    assert np.array_equal(packed, want.astype(np.uint8))


@pytest.mark.parametrize("numel,gs", [(100, 8), (1000, 32), (37, 16)])
def test_e8b_padding_of_unaligned_sizes(numel, gs):
    rng = np.random.default_rng(numel)
    w = (rng.standard_normal(numel) * 0.02).astype(np.float32)
    packed, s16, _ = O.e8b_encode(w, gs)
    padded = numel + (-numel) % gs
    assert packed.size == padded // 4 and s16.size == padded // gs
    wp = np.concatenate([w, np.zeros(padded - numel, np.float32)])
    p2, s2, _ = O.e8b_encode(wp, gs)  # F.pad semantics: the same as explicit zeros
    assert np.array_equal(packed, p2) and np.array_equal(s16, s2)


def test_e8b_rowwise_equals_whole_matrix():
    # tests/test_streaming_e8.py:15-39 of the reference, bitrate 2.0
    rng = np.random.default_rng(410)
    w = rng.standard_normal((12, 64)).astype(np.float32)
    whole, ws, _ = O.e8b_encode(w, 32)
    parts = [O.e8b_encode(w[r:r + 5], 32) for r in range(0, 12, 5)]
    assert np.array_equal(whole, np.concatenate([p[0] for p in parts]))
    assert np.array_equal(ws, np.concatenate([p[1] for p in parts]))


@pytest.mark.parametrize("dtype", [O.DT_F32, O.DT_F16, O.DT_BF16])
def test_e8b_decode_rule_matches_torch(dtype):
    rng = np.random.default_rng(50 + dtype)
    n, gs = 64 * 96, 8
    packed = rng.integers(0, 256, n // 4, dtype=np.uint8)
    s = (np.abs(rng.standard_normal(n // gs)) * 0.05).astype(np.float16)
    s[:7] = np.array([65504, 1e-7, 0, 3e-5, 6.1e-5, 1.0, 40000], dtype=np.float16)
    ours = O.e8b_decode(packed, s.view(np.uint16), n, gs, dtype)
    pk = torch.from_numpy(packed.astype(np.int64))
    codes = torch.stack([(pk >> (2 * j)) & 3 for j in range(4)], dim=-1).view(-1, gs)
    tdt = {O.DT_F32: torch.float32, O.DT_F16: torch.float16, O.DT_BF16: torch.bfloat16}[dtype]
    ref = ((codes.to(tdt) - 1.5) * torch.from_numpy(s).to(tdt).view(-1, 1)).reshape(-1)
    if dtype == O.DT_F32:
        assert np.array_equal(_bits(ours), _bits(ref.numpy()))
    else:
        assert np.array_equal(ours, ref.view(torch.int16).numpy().view(np.uint16))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("M,N,K,gs", [(2, 128, 64, 8), (3, 96, 256, 32), (1, 64, 1024, 8)])
def test_e8b_gemm_f64_matches_reference_fused_cpp(M, N, K, gs):
    rng = np.random.default_rng(M * 7 + K + gs)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    packed, s16, _ = O.e8b_encode(w, gs)
    ours = O.e8b_gemm_f64(x, packed, s16, b, N, K, gs)
    ref = O.ref_e8_fused_fwd(x, packed, O.f16_bits_to_f32(s16), b, N, K, gs)
    assert np.max(np.abs(ours - ref)) < 1e-4


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_e8b_gemm_bwd_f64_matches_reference_fused_cpp():
    rng = np.random.default_rng(19)
    M, N, K = 3, 80, 128
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    gy = rng.standard_normal((M, N)).astype(np.float32)
    packed, s16, _ = O.e8b_encode(w, 8)
    ours = O.e8b_gemm_bwd_f64(gy, packed, s16, N, K, 8)
    ref = O.ref_e8_fused_bwd_dx(gy, packed, O.f16_bits_to_f32(s16), N, K, 8)
    assert np.max(np.abs(ours - ref)) < 1e-4
