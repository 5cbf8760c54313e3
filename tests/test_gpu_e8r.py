"""GPU parity of the 1-bit Root-E8 path (RootE8LatticePacker, lattice.py:426-533).

Bars: codes, scales and decoded weights bit-exact with the CPU oracle (which is pinned
bit for bit to torch's evaluation of the reference's expression, tests/test_oracle_e8r.py);
fused forward / backward dX within max relative error 1e-2 of the fp64 oracle for bf16 /
fp16 activations and abs 1e-4 for fp32."""

import numpy as np
import pytest
import torch
import torch.nn as nn

import ojasx_amd
from ojasx_amd import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
DT_CODE = {torch.float32: O.DT_F32, torch.float16: O.DT_F16, torch.bfloat16: O.DT_BF16}
REL_TOL = 1e-2
ABS_TOL_F32 = 1e-4


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _rel_err(y, ref):
    return float(np.abs(y.detach().float().cpu().numpy() - ref).max() /
                 max(np.abs(ref).max(), 1e-30))


def _weights(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(*shape, generator=g) * 0.02
    idx = torch.randperm(w.numel(), generator=g)[: max(1, w.numel() // 1000)]
    w.view(-1)[idx] = 0.16 * torch.sign(torch.randn(idx.numel(), generator=g))
    return w.to(dtype)


@pytest.mark.parametrize("gs", [8, 16, 24, 32, 40, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_e8r_encode_bit_exact(gs, dtype):
    w = _weights((96, 384), gs * 7 + dtype.itemsize, dtype)
    w[:2] = 0
    print(f"e8r encode gs={gs} {dtype}", flush=True)
    codes, scales = ops.encode1(w.to(DEV), gs)
    torch.cuda.synchronize()
    co, so, _ = O.e8r_encode(w.float().numpy(), gs)
    assert np.array_equal(codes.cpu().numpy(), co)
    assert np.array_equal(_u16(scales), so)


@pytest.mark.parametrize("shape,gs", [((7, 13), 8), ((5, 19), 16), ((3, 40), 24), ((1, 1), 8),
                                      ((33, 17), 64)])
def test_e8r_encode_padding_tail(shape, gs):
    w = torch.randn(*shape, generator=torch.Generator().manual_seed(sum(shape) + gs))
    codes, scales = ops.encode1(w.to(DEV), gs)
    torch.cuda.synchronize()
    co, so, _ = O.e8r_encode(w.numpy(), gs)
    assert np.array_equal(codes.cpu().numpy(), co)
    assert np.array_equal(_u16(scales), so)


def test_e8r_encode_large_fp16_layer():
    w = _weights((2048, 2048), 4242, torch.float16)
    print("e8r encode 2048x2048 fp16", flush=True)
    codes, scales = ops.encode1(w.to(DEV), 32)
    torch.cuda.synchronize()
    co, so, _ = O.e8r_encode(w.float().numpy(), 32)
    assert np.array_equal(codes.cpu().numpy(), co)
    assert np.array_equal(_u16(scales), so)


def _tie_heavy_weights(kind, shape, seed):
    """Weights whose 8-vectors often have equal or nearly equal magnitudes or zeros: rows of
    the code search then tie (the kernel's candidate search must defer to the full search)."""
    g = torch.Generator().manual_seed(seed)
    if kind == "levels":       # a few quantization levels: many exactly equal magnitudes
        return (torch.randint(-3, 4, shape, generator=g).float() * 0.01).to(torch.float16)
    if kind == "pruned":       # a third of the weights exactly zero
        w = torch.randn(*shape, generator=g) * 0.02
        return (w * (torch.rand(*shape, generator=g) > 0.33)).to(torch.float16)
    if kind == "near":         # equal magnitudes up to a few ulps, random signs
        sign = torch.where(torch.rand(*shape, generator=g) < 0.5, -1.0, 1.0)
        return sign * 0.02 * (1 + torch.randint(0, 4, shape, generator=g).float() * 1e-7)
    w = torch.zeros(*shape)     # "sparse": one or two nonzeros per 8-vector
    v = w.view(-1, 8)
    v[:, 0] = torch.randn(v.shape[0], generator=g) * 0.02
    v[::2, 5] = v[::2, 0]
    return w


@pytest.mark.parametrize("kind", ["levels", "pruned", "near", "sparse"])
@pytest.mark.parametrize("gs", [8, 32, 64])
def test_e8r_encode_bit_exact_with_ties(kind, gs):
    w = _tie_heavy_weights(kind, (512, 1024), 31 * gs + len(kind))
    print(f"e8r encode ties {kind} gs={gs}", flush=True)
    codes, scales = ops.encode1(w.to(DEV), gs)
    torch.cuda.synchronize()
    co, so, _ = O.e8r_encode(w.float().numpy(), gs)
    assert np.array_equal(codes.cpu().numpy(), co)
    assert np.array_equal(_u16(scales), so)


@pytest.mark.parametrize("gs", [8, 32])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_e8r_decode_bit_exact(gs, dtype):
    rng = np.random.default_rng(gs)
    codes = rng.integers(0, 256, 4096 // 8 + 5, dtype=np.uint8)
    s16 = (rng.standard_normal((4096 + 40) // gs + 1) * 0.05).astype(np.float16)
    s16[:3] = [0.0, -0.0, 6e-8]
    numel = 4096 - 3  # a ragged tail
    out = ops.decode1(torch.from_numpy(codes).to(DEV), torch.from_numpy(s16).to(DEV), numel, gs,
                      dtype)
    torch.cuda.synchronize()
    ref = O.e8r_decode(codes, s16.view(np.uint16), numel, gs, DT_CODE[dtype])
    if dtype == torch.float32:
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    else:
        assert np.array_equal(_u16(out), ref)


def _layer1(N, K, seed, gs):
    w = _weights((N, K), seed)
    codes, s16, _ = O.e8r_encode(w.numpy(), gs)
    return (torch.from_numpy(codes).to(DEV), torch.from_numpy(s16.view(np.float16).copy()).to(DEV),
            codes, s16)


@pytest.mark.parametrize("M,N,K,gs,dtype", [
    (1, 256, 512, 32, torch.bfloat16),      # decode GEMV
    (5, 130, 1024, 8, torch.float16),       # decode GEMV, ragged last tile
    (2, 256, 320, 32, torch.bfloat16),      # K % 256 != 0: MFMA kernel, small tiles
    (17, 256, 512, 16, torch.bfloat16),
    (100, 1000, 256, 64, torch.float16),
    (300, 520, 512, 32, torch.bfloat16),
    (40, 1024, 4096, 8, torch.bfloat16),     # K split
    (3, 96, 96, 32, torch.bfloat16),         # K % 64 != 0: general kernel
    (4, 64, 120, 24, torch.float16),         # group size 24: general kernel
    (6, 72, 128, 32, torch.float32),         # fp32 activations: general kernel
])
def test_e8r_fwd_matches_oracle(M, N, K, gs, dtype):
    pk, sc, pk_np, sc_np = _layer1(N, K, seed=M + N + K + gs, gs=gs)
    g = torch.Generator().manual_seed(M * 5 + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"e8r fwd M={M} N={N} K={K} gs={gs} {dtype}", flush=True)
    y = ops.e8r_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, gs)
    torch.cuda.synchronize()
    ref = O.e8r_gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, gs,
                         DT_CODE[dtype])
    assert y.shape == (M, N) and y.dtype == dtype
    if dtype == torch.float32:
        assert float(np.abs(y.cpu().numpy() - ref).max()) <= ABS_TOL_F32 * max(1.0, np.abs(ref).max())
    else:
        assert _rel_err(y, ref) <= REL_TOL


@pytest.mark.parametrize("M,N,K,gs,dtype", [
    (16, 777, 2048, 32, torch.bfloat16),    # one round pair per wave
    (16, 64, 5120, 64, torch.float16),      # pairs and a tail round
    (8, 1000, 768, 16, torch.bfloat16),     # three rounds: one wave idle
    (12, 4096, 14336, 8, torch.bfloat16),   # down-projection shape
    (1, 4096, 4096, 32, torch.bfloat16),
    (4, 16, 256, 8, torch.float16),         # a single round
])
def test_e8r_gemv_kernel_matches_oracle(M, N, K, gs, dtype):
    # M <= 16, K % 256 == 0 and gs in {8, 16, 32, 64} select the decode GEMV (weights in
    # the B operand from the value words and the code's selector words)
    pk, sc, pk_np, sc_np = _layer1(N, K, seed=2 * N + K + gs, gs=gs)
    g = torch.Generator().manual_seed(M * 11 + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"e8r gemv M={M} N={N} K={K} gs={gs} {dtype}", flush=True)
    y = ops.e8r_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, gs)
    torch.cuda.synchronize()
    ref = O.e8r_gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, gs,
                         DT_CODE[dtype])
    assert y.shape == (M, N) and y.dtype == dtype
    assert _rel_err(y, ref) <= REL_TOL


@pytest.mark.parametrize("M,N,K,gs,dtype", [
    (1, 16 * 37 + 5, 256, 32, torch.bfloat16),    # one round: three waves only load spares
    (3, 16 * 37 + 5, 1280, 8, torch.float16),     # five rounds: one wave has two
    (4, 16 * 37 + 5, 4096, 64, torch.bfloat16),   # four rounds per wave: all in flight
    (2, 16 * 37 + 5, 5120, 16, torch.bfloat16),   # five rounds per wave: a second pass
    (4, 16 * 600, 1024, 32, torch.bfloat16),      # two row tiles per workgroup
    (2, 16 * 600 + 7, 2048, 8, torch.float16),    # ... ragged last tile
])
def test_e8r_gemv_m4_pipeline_matches_oracle(M, N, K, gs, dtype):
    # M <= 4 (M = 1 only where K % 1024 != 0): the B-operand GEMV that stages activation rows
    # 0..3 and keeps four rounds per wave in flight (spare slots past a wave's last round load
    # nothing)
    pk, sc, pk_np, sc_np = _layer1(N, K, seed=3 * N + K + gs, gs=gs)
    g = torch.Generator().manual_seed(M * 13 + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"e8r gemv m4 M={M} N={N} K={K} gs={gs} {dtype}", flush=True)
    y = ops.e8r_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, gs)
    torch.cuda.synchronize()
    ref = O.e8r_gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, gs,
                         DT_CODE[dtype])
    assert y.shape == (M, N) and y.dtype == dtype
    assert _rel_err(y, ref) <= REL_TOL
    for m in range(M):  # each activation row against its own scale
        assert _rel_err(y[m:m + 1], ref[m:m + 1]) <= REL_TOL, m


@pytest.mark.parametrize("N,K,gs,dtype,bias", [
    (16 * 37 + 5, 1024, 32, torch.bfloat16, True),    # one round: three waves idle
    (16 * 37 + 5, 3072, 8, torch.float16, True),      # three rounds, one per wave
    (16 * 300 + 9, 5120, 16, torch.bfloat16, False),  # wave 0: a last pair
    (1000, 9216, 64, torch.float16, True),            # wave 0: a round pair, then a last round
    (4096, 14336, 32, torch.bfloat16, True),          # down projection: the loop and a pair
])
def test_e8r_post_scaled_m1_matches_oracle(N, K, gs, dtype, bias):
    # M = 1, K % 1024 == 0: the post-scaled GEMV (a code byte's eight coordinates from the
    # table, the group scale applied to fp32 partial sums), one row tile per workgroup and
    # rounds u = w, w + 4, ... per wave
    pk, sc, pk_np, sc_np = _layer1(N, K, seed=5 * N + K + gs, gs=gs)
    g = torch.Generator().manual_seed(K + gs)
    x = torch.randn(1, K, generator=g).to(dtype)
    b = torch.randn(N, generator=g).to(dtype) if bias else None
    print(f"e8r post-scaled M=1 N={N} K={K} gs={gs} {dtype} bias={bias}", flush=True)
    y = ops.e8r_linear(x.to(DEV), pk, sc, b.to(DEV) if bias else None, N, K, gs)
    torch.cuda.synchronize()
    ref = O.e8r_gemm_f64(x.float().numpy(), pk_np, sc_np, b.float().numpy() if bias else None,
                         N, K, gs, DT_CODE[dtype])
    assert y.shape == (1, N) and y.dtype == dtype
    assert _rel_err(y, ref) <= REL_TOL
    # the same weights through the B-operand GEMV (two activation rows) agree row by row
    x2 = torch.cat([x, x]).to(DEV)
    y2 = ops.e8r_linear(x2, pk, sc, b.to(DEV) if bias else None, N, K, gs)
    torch.cuda.synchronize()
    assert _rel_err(y2[1:2], ref) <= REL_TOL


def test_e8r_prefill_large_shape_against_decoded_matmul():
    N, K, M, gs = 14336, 4096, 512, 32
    gw = torch.Generator(device=DEV).manual_seed(77)
    w = torch.randn(N, K, generator=gw, device=DEV) * 0.02
    codes, scales = ops.encode1(w, gs)
    del w
    x = torch.randn(M, K, generator=gw, device=DEV).to(torch.bfloat16)
    print("e8r prefill gate_up M=512", flush=True)
    y = ops.e8r_linear(x, codes, scales, None, N, K, gs)
    wdq = ops.decode1(codes, scales, N * K, gs, torch.bfloat16).view(N, K).float()
    ref = x.float() @ wdq.t().contiguous()
    torch.cuda.synchronize()
    assert ((y.float() - ref).abs().max() / ref.abs().max()).item() <= REL_TOL
    rows = [0, 255, 511]
    ref64 = O.e8r_gemm_f64(x[rows].float().cpu().numpy(), codes.cpu().numpy(), _u16(scales), None,
                           N, K, gs, O.DT_BF16)
    assert _rel_err(y[rows], ref64) <= REL_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(1, 128, 256), (7, 96, 512)])
def test_e8r_bwd_dx_matches_oracle(dtype, M, N, K):
    pk, sc, pk_np, sc_np = _layer1(N, K, seed=N + K + 9, gs=32)
    gy = torch.randn(M, N, generator=torch.Generator().manual_seed(M)).to(dtype)
    gx = ops.e8r_linear_bwd_dx(gy.to(DEV), pk, sc, N, K, 32)
    torch.cuda.synchronize()
    ref = O.e8r_gemm_bwd_f64(gy.float().numpy(), pk_np, sc_np, N, K, 32, DT_CODE[dtype])
    if dtype == torch.float32:
        assert float(np.abs(gx.cpu().numpy() - ref).max()) <= ABS_TOL_F32 * max(1.0, np.abs(ref).max())
    else:
        assert _rel_err(gx, ref) <= REL_TOL


def test_e8r_layer_with_hadamard_and_lora_forward_backward():
    # the reference's test_e8_lattice_linear_1bit_and_hadamard, on the GPU path: the layer
    # output equals x @ unpack_weights()^T + bias + LoRA, and gradients flow to x and LoRA
    torch.manual_seed(0)
    lin = nn.Linear(64, 64, bias=True).to(DEV)
    layer = ojasx_amd.E8LatticeLinear.from_linear(lin, bitrate=1.0, rank=8, group_size=32,
                                                  use_hadamard=True)
    assert layer.use_hadamard and layer.bitrate == 1.0
    assert layer.packed_weight.shape == (64 * 64 // 8,)
    with torch.no_grad():
        layer.lora_B.normal_(0, 0.02)
    x = torch.randn(4, 16, 64, device=DEV, requires_grad=True)
    out = layer(x)
    assert out.shape == (4, 16, 64)
    w = layer.unpack_weights(torch.float32)
    ref = x @ w.t() + layer.bias + layer.scaling * ((x @ layer.lora_A) @ layer.lora_B)
    assert torch.allclose(out, ref, atol=1e-4, rtol=1e-4)
    out.sum().backward()
    assert x.grad is not None and x.grad.shape == x.shape
    gref = torch.ones(4, 16, 64, device=DEV) @ (w + (layer.scaling * layer.lora_A @ layer.lora_B).t())
    assert torch.allclose(x.grad, gref, atol=1e-3, rtol=1e-3)
    assert layer.lora_A.grad is not None and layer.lora_B.grad is not None


def test_e8r_pack_model_and_rowwise_packing():
    class Toy(nn.Module):
        def __init__(self):
            super().__init__()
            self.fc1 = nn.Linear(64, 64)
            self.fc2 = nn.Linear(64, 32)

        def forward(self, x):
            return self.fc2(torch.relu(self.fc1(x)))

    model = Toy().to(DEV)
    packed = ojasx_amd.pack_model_e8(model, bitrate=1.0, rank=4, group_size=32, use_hadamard=True)
    assert isinstance(packed.fc1, ojasx_amd.E8LatticeLinear) and packed.fc1.bitrate == 1.0
    assert packed(torch.randn(2, 64, device=DEV)).shape == (2, 32)
    # streaming row-block packing is byte-exact to whole-matrix packing (the reference test
    # tests/test_streaming_e8.py:15-39 at bitrate 1.0)
    torch.manual_seed(410)
    weight = torch.randn(12, 64)
    for had in (False, True):
        src = ojasx_amd.fwht_block32(weight) if had else weight
        codes, scales, _ = ojasx_amd.RootE8LatticePacker.pack(src, group_size=32)
        rc, rs = ojasx_amd.pack_weight_rowwise(weight, bitrate=1.0, group_size=32, row_block=5,
                                               use_hadamard=had)
        assert torch.equal(rc, codes) and torch.equal(rs, scales)
        co, so, _ = O.e8r_encode(src.numpy(), 32)
        assert np.array_equal(codes.numpy(), co) and np.array_equal(_u16(scales), so)
