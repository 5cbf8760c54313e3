"""Pins the CPU oracle (oracle/e8t_oracle.c) before anything is compared to it.

Each check is independent of the oracle's own formulas:
  * number conversions      -> numpy / torch library conversions
  * group scale             -> torch.norm(...) / math.sqrt(gs) + 1e-8, the exact
                               expression of lattice.py:356 evaluated by torch
  * codebook                -> the reference's own C++ LUT (oracle/_ref), built
                               from ojasx_math_core.hpp:549-573
  * nearest-point rule      -> exhaustive search over all 3,281 codewords, and
                               hand-derived tie cases (tests/golden/known_answers.json)
  * byte layout / sizes     -> closed form and the reference tests' invariants
                               (tests/test_sub2bit_lattice.py:40-62,
                               tests/test_streaming_e8.py:15-39 of the reference)
  * dequant-matmul          -> the reference's own fused C++ GEMV (oracle/_ref),
                               tolerance of tests/test_fused_e8_gemm.py:153-182
"""

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


# ---------------------------------------------------------------- conversions

def _special_f32():
    rng = np.random.default_rng(5)
    vals = [
        rng.standard_normal(200000).astype(np.float32) * np.float32(0.02),
        rng.standard_normal(50000).astype(np.float32) * np.float32(3e4),
        (rng.random(50000) * np.float32(7e-5)).astype(np.float32),  # fp16 subnormal range
        (rng.random(50000) * np.float32(1e-7)).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 1e-45],
                 dtype=np.float32),
    ]
    # every fp16 value, and the exact midpoints between neighbours (ties)
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    vals += [h, -h, mids, -mids]
    return np.concatenate(vals)


def test_f32_to_f16_matches_numpy():
    x = _special_f32()
    ours = O.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):  # values past the fp16 range round to +-inf
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f32_to_f16_matches_torch():
    x = _special_f32()
    ours = O.f32_to_f16_bits(x)
    ref = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f32_to_bf16_matches_torch():
    x = _special_f32()
    ours = O.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


# ---------------------------------------------------------------- scale

@pytest.mark.parametrize("gs", [16, 32, 48, 64, 128, 256])
def test_group_scale_matches_torch_norm_expression(gs):
    g = torch.Generator().manual_seed(100 + gs)
    w = torch.randn(20000, gs, generator=g) * 0.02
    idx = torch.randperm(w.numel(), generator=g)[: w.numel() // 1000]
    w.view(-1)[idx] = 0.16 * torch.sign(torch.randn(idx.numel(), generator=g))
    w[:50] = 0.0  # zero groups -> s = 1e-8
    ref = (torch.norm(w, dim=-1) / math.sqrt(gs) + 1e-8).numpy()
    ours = O.group_scales(w.numpy())
    assert np.array_equal(_bits(ours), _bits(ref))
    ref16 = torch.from_numpy(ref).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_f16_bits(ours), ref16)


def test_group_scale_from_fp16_source():
    # C4 stores weights in fp16; the pack casts them exactly to fp32 first (lattice.py:350)
    g = torch.Generator().manual_seed(7)
    w = (torch.randn(30000, 32, generator=g) * 0.02).half().float()
    ref = (torch.norm(w, dim=-1) / math.sqrt(32) + 1e-8).numpy()
    assert np.array_equal(_bits(O.group_scales(w.numpy())), _bits(ref))


# ---------------------------------------------------------------- codebook

def test_codebook_closed_form_properties():
    cb = O.codebook()
    assert cb.shape == (3281, 8)
    assert set(np.unique(cb)) <= {-1, 0, 1}
    assert np.all(cb.sum(axis=1) % 2 == 0)
    # all distinct and complete: |D8 cap {-1,0,1}^8| = (3^8 + 1) / 2 = 3281
    assert len({tuple(r) for r in cb}) == 3281
    # increasing raw order
    raw = ((cb.astype(np.int64) + 1) * 3 ** np.arange(8)).sum(axis=1)
    assert np.all(np.diff(raw) > 0)
    assert np.array_equal(raw, 2 * np.arange(3281))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_codebook_matches_reference_cpp_lut():
    assert np.array_equal(O.codebook(), O.ref_codebook())


# ---------------------------------------------------------------- nearest point

def _brute_force(v: np.ndarray, cb: np.ndarray):
    """Exact squared distances (float64) to all codewords; returns best, margin."""
    v64 = v.astype(np.float64)
    d = ((cb[None, :, :].astype(np.float64) - v64[:, None, :]) ** 2).sum(axis=2)
    order = np.argsort(d, axis=1, kind="stable")
    best = order[:, 0]
    rows = np.arange(v.shape[0])
    margin = d[rows, order[:, 1]] - d[rows, best]
    return best, margin


def test_quantize8_is_nearest_codeword_on_random_vectors():
    cb = O.codebook()
    rng = np.random.default_rng(11)
    chunks = [
        rng.standard_normal((8000, 8)).astype(np.float32),
        (rng.standard_normal((8000, 8)) * 0.6).astype(np.float32),
        (rng.random((8000, 8)) * 3 - 1.5).astype(np.float32),
    ]
    v = np.concatenate(chunks)
    ours = O.quantize8_many(v)
    best, margin = _brute_force(v, cb)
    clear = margin > 1e-5
    assert clear.mean() > 0.999
    assert np.array_equal(ours[clear], best[clear])


def test_encode_codes_are_nearest_codewords_of_w_over_s():
    # the real distribution: N(0, 0.02) groups with +-8 sigma outliers
    rng = np.random.default_rng(12)
    w = (rng.standard_normal(32 * 4000) * 0.02).astype(np.float32)
    idx = rng.choice(w.size, w.size // 1000, replace=False)
    w[idx] = np.float32(0.16) * np.sign(rng.standard_normal(idx.size)).astype(np.float32)
    packed, scales16, s32 = O.encode(w, 32)
    codes = O.unpack_codes(packed)
    v = (w.reshape(-1, 32) / s32[:, None]).astype(np.float32).reshape(-1, 8)
    best, margin = _brute_force(v, O.codebook())
    clear = margin > 1e-5
    assert clear.mean() > 0.999
    assert np.array_equal(codes[clear], best[clear])


def test_quantize8_known_answers():
    with open(os.path.join(GOLDEN, "known_answers.json")) as f:
        ka = json.load(f)
    for case in ka["quantize8"]:
        v = np.array([float(t) for t in case["v"]], dtype=np.float32)
        code, q = O.quantize8(v)
        assert code == case["code"], case["why"]
        assert q.tolist() == case["q"], case["why"]


def test_encode_group_known_answers():
    with open(os.path.join(GOLDEN, "known_answers.json")) as f:
        ka = json.load(f)
    for case in ka["groups"]:
        w = np.array(case["w"], dtype=np.float32)
        packed, s16, s32 = O.encode(w, case["gs"])
        assert O.unpack_codes(packed).tolist() == case["codes"], case["why"]
        assert int(s16[0]) == case["scale_f16"], case["why"]
        assert int(_bits(s32)[0]) == int(case["scale_f32_hex"], 16), case["why"]


# ---------------------------------------------------------------- layout

def _minus_zero_group() -> np.ndarray:
    # the first weight is fp32's smallest negative subnormal; its quotient by the group scale
    # (~2.12) rounds to -0, and the parity fix then flips coordinate 0 (pen 1, the first
    # minimum).  Only fp32 inputs reach -0: a bf16/fp16 subnormal over a scale that fp16 can
    # hold still has a nonzero quotient.
    w = np.zeros(32, dtype=np.float32)
    w[0] = -np.float32(1e-45)
    w[1] = 12.0
    return w


def test_encode_minus_zero_quotient_flips_up():
    # lattice.py:361-365: alt = +1 where v >= 0, and -0 >= 0 holds, so coordinate 0 becomes
    # +1: coords [1, 1, 0, ...] -> raw = 2 + 2*3 + (3280 - 1 - 3) = 3284 -> code 1642; the
    # three all-zero 8-vectors have code 1640 (Appendix-A closed form)
    p, _, _ = O.encode(_minus_zero_group()[None, :], 32)
    want = np.array([b for c0, c1 in ((1642, 1640), (1640, 1640))
                     for b in (c0 & 0xFF, ((c0 >> 8) & 0xF) | ((c1 & 0xF) << 4), (c1 >> 4) & 0xFF)],
                    dtype=np.uint8)
    assert np.array_equal(p, want), p
    # the reference's expressions evaluated by torch: v[0] is -0 and its alt is +1
    w = torch.from_numpy(_minus_zero_group())
    sc = torch.norm(w) / math.sqrt(32) + 1e-8
    v = w.view(4, 8) / sc
    assert str(float(v[0, 0])) == "-0.0"
    q = torch.clamp(torch.round(v), -1, 1)
    alt = torch.where(q == 0, torch.where(v >= 0, 1.0, -1.0), 0.0)
    assert float(alt[0, 0]) == 1.0


def test_packed_sizes_match_reference_invariants():
    # reference tests/test_sub2bit_lattice.py:40-62: 64x128 at gs 32
    rng = np.random.default_rng(99)
    w = rng.standard_normal((64, 128)).astype(np.float32)
    packed, scales, _ = O.encode(w, 32)
    assert packed.size == int(w.size * 1.5 / 8)
    assert scales.size == w.size // 32
    rec = O.decode(packed, scales, w.size, 32).reshape(w.shape)
    cos = float(np.dot(rec.ravel(), w.ravel()) / (np.linalg.norm(rec) * np.linalg.norm(w)))
    assert cos > 0.70


def test_byte_layout_closed_form():
    rng = np.random.default_rng(3)
    w = rng.standard_normal(16 * 50).astype(np.float32)
    packed, scales, s32 = O.encode(w, 16)
    codes = O.unpack_codes(packed)
    # re-pack by the closed form of lattice.py:379-383
    c0, c1 = codes[0::2], codes[1::2]
    b = np.stack([c0 & 0xFF, ((c0 >> 8) & 0x0F) | ((c1 & 0x0F) << 4), (c1 >> 4) & 0xFF], 1)
    assert np.array_equal(b.reshape(-1).astype(np.uint8), packed)
    # 12-bit little-endian bit stream: code t sits at bits [12t, 12t+12)
    bits = np.unpackbits(packed, bitorder="little")
    for t in range(0, codes.size, 7):
        val = int(sum(int(bits[12 * t + i]) << i for i in range(12)))
        assert val == codes[t]


@pytest.mark.parametrize("shape,gs", [((7, 13), 16), ((5, 19), 32), ((3, 40), 48)])
def test_padding_and_decode_of_unaligned_shapes(shape, gs):
    # reference tests/test_ojasx_exhaustive.py:301-320 shapes
    rng = np.random.default_rng(sum(shape))
    w = rng.standard_normal(shape).astype(np.float32)
    n = w.size
    p = O.padded(n, gs)
    assert p % gs == 0 and p - n < gs
    packed, scales, s32 = O.encode(w, gs)
    assert packed.size == p * 3 // 16 and scales.size == p // gs
    rec = O.decode(packed, scales, n, gs)
    codes = O.unpack_codes(packed)
    cb = O.codebook().astype(np.float32)
    full = (cb[codes].reshape(-1, gs) * O.f16_bits_to_f32(scales)[:, None]).reshape(-1)
    assert np.array_equal(_bits(rec), _bits(full[:n]))


def test_group_size_coercion():
    # lattice.py:346-347: gs not a positive multiple of 16 -> 16
    assert O.effective_gs(8) == 16
    assert O.effective_gs(24) == 16
    assert O.effective_gs(0) == 16
    assert O.effective_gs(32) == 32
    assert O.effective_gs(48) == 48


def test_rowwise_encoding_equals_whole_matrix():
    # reference tests/test_streaming_e8.py:15-39: row blocks with whole groups pack
    # to the same bytes as the flat matrix
    rng = np.random.default_rng(410)
    w = rng.standard_normal((12, 64)).astype(np.float32)
    pw, sw, _ = O.encode(w, 32)
    parts = [O.encode(w[r:r + 5], 32) for r in range(0, 12, 5)]
    assert np.array_equal(np.concatenate([p[0] for p in parts]), pw)
    assert np.array_equal(np.concatenate([p[1] for p in parts]), sw)


@pytest.mark.parametrize("dtype", [O.DT_F16, O.DT_BF16])
def test_decode_low_precision_rule(dtype):
    # lattice.py:414-418: coords.to(dtype) * scales.to(dtype), evaluated by torch
    rng = np.random.default_rng(21 + dtype)
    w = (rng.standard_normal(64 * 96) * 0.02).astype(np.float32)
    packed, scales, _ = O.encode(w, 32)
    ours = O.decode(packed, scales, w.size, 32, dtype)
    codes = torch.from_numpy(O.unpack_codes(packed).astype(np.int64))
    cb = torch.from_numpy(O.codebook())
    tdt = torch.float16 if dtype == O.DT_F16 else torch.bfloat16
    s = torch.from_numpy(scales.view(np.float16).copy())
    ref = (cb[codes].view(-1, 32).to(tdt) * s.to(tdt).view(-1, 1)).reshape(-1)
    assert np.array_equal(ours, ref.view(torch.int16).numpy().view(np.uint16))


# ---------------------------------------------------------------- matmul reference

@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("M,N,K", [(2, 128, 64), (3, 96, 256), (1, 64, 1024)])
def test_gemm_f64_matches_reference_fused_cpp(M, N, K):
    rng = np.random.default_rng(M * 7 + K)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    packed, s16, _ = O.encode(w, 32)
    ours = O.gemm_f64(x, packed, s16, b, N, K, 32)
    ref = O.ref_fused_fwd(x, packed, O.f16_bits_to_f32(s16), b, N, K, 32)
    assert np.max(np.abs(ours - ref)) < 1e-4


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_gemm_bwd_f64_matches_reference_fused_cpp():
    rng = np.random.default_rng(17)
    M, N, K = 3, 80, 128
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    gy = rng.standard_normal((M, N)).astype(np.float32)
    packed, s16, _ = O.encode(w, 32)
    ours = O.gemm_bwd_f64(gy, packed, s16, N, K, 32)
    ref = O.ref_fused_bwd_dx(gy, packed, O.f16_bits_to_f32(s16), N, K, 32)
    assert np.max(np.abs(ours - ref)) < 1e-4


def test_gemm_f64_matches_torch_portable_restatement():
    from oracle import portable

    rng = np.random.default_rng(23)
    M, N, K = 4, 72, 96
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    packed, s16, _ = O.encode(w, 32)
    y = portable.linear(torch.from_numpy(x), torch.from_numpy(packed),
                        torch.from_numpy(s16.view(np.float16).copy()), None, N, K)
    ref = O.gemm_f64(x, packed, s16, None, N, K, 32)
    assert np.max(np.abs(y.numpy() - ref)) < 1e-4
