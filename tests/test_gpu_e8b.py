"""GPU parity of the 2-bit E8 path (E8LatticePacker, lattice.py:209-279).

Bars: codes, scales and decoded weights bit-exact with the CPU oracle (byte work);
fused forward / backward dX within max relative error 1e-2 of the fp64 oracle for
bf16 / fp16 activations and abs 1e-4 for fp32 at the reference test's shapes
(tests/test_fused_e8_gemm.py of the reference)."""

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

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


def _outliers(w, g, frac=1000, sigma=0.16):
    idx = torch.randperm(w.numel(), generator=g)[: max(1, w.numel() // frac)]
    signs = torch.where(torch.rand(idx.numel(), generator=g) < 0.5, -1.0, 1.0)
    w.view(-1)[idx] = (sigma * signs).to(w.dtype)
    return w


def _rel_err(y, ref):
    return float(np.abs(y.detach().float().cpu().numpy() - ref).max() /
                 max(np.abs(ref).max(), 1e-30))


@pytest.mark.parametrize("gs", [8, 16, 24, 32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_e8b_encode_bit_exact(gs, dtype):
    g = torch.Generator().manual_seed(gs * 11 + int(dtype.itemsize))
    w = _outliers(torch.randn(96, 384, generator=g) * 0.02, g).to(dtype)
    w[:2] = 0  # zero groups
    print(f"e8b encode gs={gs} {dtype}", flush=True)
    packed, scales = ops.encode2(w.to(DEV), gs)
    torch.cuda.synchronize()
    po, so, _ = O.e8b_encode(w.float().numpy(), gs)
    assert np.array_equal(_u16(scales), so)
    assert np.array_equal(packed.cpu().numpy(), po)


@pytest.mark.parametrize("shape,gs", [((7, 13), 8), ((5, 19), 16), ((3, 40), 24), ((1, 1), 8),
                                      ((33, 17), 64)])
def test_e8b_encode_padding_tail(shape, gs):
    g = torch.Generator().manual_seed(sum(shape) + gs)
    w = torch.randn(*shape, generator=g)
    packed, scales = ops.encode2(w.to(DEV), gs)
    torch.cuda.synchronize()
    po, so, _ = O.e8b_encode(w.numpy(), gs)
    assert np.array_equal(packed.cpu().numpy(), po) and np.array_equal(_u16(scales), so)


def test_e8b_encode_large_fp16_layer_with_outliers():
    # a gate/up-sized fp16 layer with 0.1% +-8 sigma outliers at the default group size 8
    g = torch.Generator().manual_seed(9001)
    w = _outliers((torch.randn(14336, 4096, generator=g) * 0.02), g).half()
    print("e8b encode 14336x4096 fp16", flush=True)
    packed, scales = ops.encode2(w.to(DEV), 8)
    torch.cuda.synchronize()
    po, so, _ = O.e8b_encode(w.float().numpy(), 8)
    assert np.array_equal(_u16(scales), so)
    assert np.array_equal(packed.cpu().numpy(), po)


@pytest.mark.parametrize("gs", [8, 32])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_e8b_decode_bit_exact(gs, dtype):
    rng = np.random.default_rng(gs + int(dtype.itemsize))
    numel = 96 * 200 + (13 if gs == 8 else 0)  # a ragged tail at gs 8
    padded = numel + (-numel) % gs
    packed = rng.integers(0, 256, padded // 4, dtype=np.uint8)
    s = (np.abs(rng.standard_normal(padded // gs)) * 0.05).astype(np.float16)
    s[:5] = np.array([65504, 1e-7, 0, 6.1e-5, 40000], dtype=np.float16)
    out = ops.decode2(torch.from_numpy(packed).to(DEV),
                      torch.from_numpy(s).to(DEV), numel, gs, dtype)
    ref = O.e8b_decode(packed, s.view(np.uint16), numel, gs, DT_CODE[dtype])
    if dtype == torch.float32:
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    else:
        assert np.array_equal(_u16(out), ref)


def _layer2(N, K, seed, gs=8, scale=0.02):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * scale
    packed, s16, _ = O.e8b_encode(w.numpy(), gs)
    return (torch.from_numpy(packed).to(DEV),
            torch.from_numpy(s16.view(np.float16).copy()).to(DEV), packed, s16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,N,K,gs", [(1, 256, 512, 8), (3, 128, 256, 32), (16, 96, 1024, 8),
                                      (64, 192, 512, 16), (130, 64, 256, 8), (5, 40, 96, 8),
                                      (2, 33, 20, 4)])
def test_e8b_fwd_matches_oracle(dtype, M, N, K, gs):
    pk, sc, pk_np, sc_np = _layer2(N, K, seed=M * 17 + N + gs, gs=gs) if gs % 8 == 0 else \
        _layer2_any(N, K, gs)
    g = torch.Generator().manual_seed(K + gs)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"e8b fwd M={M} N={N} K={K} gs={gs} {dtype}", flush=True)
    y = ops.e8_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, gs)
    ref = O.e8b_gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, gs,
                         DT_CODE[dtype])
    assert y.shape == (M, N) and y.dtype == dtype
    if dtype == torch.float32:
        assert float(np.abs(y.cpu().numpy() - ref).max()) <= ABS_TOL_F32 * max(1.0, np.abs(ref).max())
    else:
        assert _rel_err(y, ref) <= REL_TOL


def _layer2_any(N, K, gs):
    # group sizes the packer rejects but the native op accepts (multiples of 4): random
    # codes and scales in the 2-bit layout
    rng = np.random.default_rng(N * K + gs)
    padded = N * K + (-(N * K)) % gs
    packed = rng.integers(0, 256, padded // 4, dtype=np.uint8)
    s16 = (np.abs(rng.standard_normal(padded // gs)) * 0.02).astype(np.float16).view(np.uint16)
    return (torch.from_numpy(packed).to(DEV),
            torch.from_numpy(s16.view(np.float16).copy()).to(DEV), packed, s16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(1, 128, 256), (7, 96, 512), (64, 80, 128)])
def test_e8b_bwd_dx_matches_oracle(dtype, M, N, K):
    pk, sc, pk_np, sc_np = _layer2(N, K, seed=N + K + 5)
    gy = torch.randn(M, N, generator=torch.Generator().manual_seed(M)).to(dtype)
    gx = ops.e8_linear_bwd_dx(gy.to(DEV), pk, sc, N, K, 8)
    ref = O.e8b_gemm_bwd_f64(gy.float().numpy(), pk_np, sc_np, N, K, 8, DT_CODE[dtype])
    if dtype == torch.float32:
        assert float(np.abs(gx.cpu().numpy() - ref).max()) <= ABS_TOL_F32 * max(1.0, np.abs(ref).max())
    else:
        assert _rel_err(gx, ref) <= REL_TOL


@pytest.mark.parametrize("M", [1, 4, 16])
def test_e8b_decode_gemv_8b_shape(M):
    # a q/o-shaped 2-bit layer at the default group size 8, bf16 activations
    N = K = 4096
    pk, sc, pk_np, sc_np = _layer2(N, K, seed=8200)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(8300 + M)).to(torch.bfloat16)
    y = ops.e8_linear(x.to(DEV), pk, sc, None, N, K, 8)
    ref = O.e8b_gemm_f64(x.float().numpy(), pk_np, sc_np, None, N, K, 8, O.DT_BF16)
    assert _rel_err(y, ref) <= REL_TOL


def test_e8b_layer_matches_reference_fused_test():
    # the reference's tests/test_fused_e8_gemm.py pattern at bitrate 2.0 (fp32, abs 1e-4)
    torch.manual_seed(42)
    ref_linear = nn.Linear(128, 256, bias=True).to(DEV)
    layer = ojasx_amd.E8LatticeLinear.from_linear(ref_linear, rank=4, bitrate=2.0, group_size=8)
    assert layer.packed_weight.numel() == 128 * 256 // 4
    x = torch.randn(3, 8, 128, device=DEV)
    w_unpacked = layer.unpack_weights(dtype=x.dtype)
    expected = F.linear(x, w_unpacked, layer.bias)
    expected = expected + layer.scaling * ((x @ layer.lora_A) @ layer.lora_B)
    out = layer.forward_fused(x)
    assert float((out - expected).detach().abs().max()) < 1e-4
    # the packed bytes are the oracle's
    po, so, _ = O.e8b_encode(ref_linear.weight.detach().cpu().numpy(), 8)
    assert np.array_equal(layer.packed_weight.cpu().numpy(), po)


def test_e8b_layer_backward_and_lora_grads():
    torch.manual_seed(3)
    lin = nn.Linear(64, 48).to(DEV)
    layer = ojasx_amd.E8LatticeLinear.from_linear(lin, rank=2, bitrate=2.0, group_size=8)
    with torch.no_grad():
        layer.lora_B.normal_()
    x = torch.randn(5, 64, device=DEV, requires_grad=True)
    layer(x).square().sum().backward()
    w = layer.unpack_weights(torch.float32)
    x2 = x.detach().clone().requires_grad_(True)
    ref = F.linear(x2, w, layer.bias.detach()) + layer.scaling * ((x2 @ layer.lora_A.detach()) @ layer.lora_B.detach())
    ref.square().sum().backward()
    assert torch.allclose(x.grad, x2.grad, atol=1e-4, rtol=1e-4)
    assert layer.lora_A.grad is not None and layer.bias.grad is not None


def test_e8b_native_schema_ops_and_rowwise_packing():
    torch.manual_seed(410)
    weight = torch.randn(12, 64)
    whole, ws, _ = ojasx_amd.E8LatticePacker.pack(weight, group_size=32)
    pk, sc = ojasx_amd.pack_weight_rowwise(weight, bitrate=2.0, group_size=32, row_block=5)
    assert torch.equal(pk, whole) and torch.equal(sc, ws)
    x = torch.randn(4, 64, device=DEV)
    y = ops.fused_e8_gemm_fwd(x, whole.to(DEV).view(12, 16), ws.to(DEV), None, 32)
    w = ojasx_amd.E8LatticePacker.unpack(whole, ws, (12, 64)).to(DEV)
    assert torch.allclose(y, x @ w.t(), atol=1e-4)
    gy = torch.randn(4, 12, device=DEV)
    gx = ops.fused_e8_gemm_bwd_dx(gy, whole.to(DEV).view(12, 16), ws.to(DEV), 64, 32)
    assert torch.allclose(gx, gy @ w, atol=1e-4)
    with pytest.raises(RuntimeError, match="in_features / 4"):
        ops.fused_e8_gemm_fwd(x, whole[:96].to(DEV).view(12, 8), ws.to(DEV), None, 32)
    with pytest.raises(RuntimeError, match="block_scales"):
        ops.fused_e8_gemm_fwd(x, whole.to(DEV).view(12, 16), ws[:20].to(DEV), None, 32)


@pytest.mark.parametrize("M,N,K,gs,dtype", [
    (1, 4100, 3072, 8, torch.bfloat16),    # odd round count, ragged last tile
    (2, 1000, 1024, 16, torch.float16),    # one round
    (3, 777, 2048, 32, torch.bfloat16),
    (4, 64, 5120, 64, torch.bfloat16),     # five rounds, one workgroup
    (4, 4096, 14336, 8, torch.bfloat16),   # down-projection shape
    (1, 16, 1024, 8, torch.float16),
])
def test_e8b_gemv_kernel_matches_oracle(M, N, K, gs, dtype):
    # M <= 4, K % 1024 == 0 and gs in {8, 16, 32, 64} select the 2-bit MFMA decode GEMV
    pk, sc, pk_np, sc_np = _layer2(N, K, seed=N + K + gs, gs=gs)
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"e8b gemv M={M} N={N} K={K} gs={gs} {dtype}", flush=True)
    y = ops.e8_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, gs)
    torch.cuda.synchronize()
    ref = O.e8b_gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, gs,
                         DT_CODE[dtype])
    assert _rel_err(y, ref) <= REL_TOL


@pytest.mark.parametrize("M,N,K,gs,dtype", [
    (5, 4100, 1024, 8, torch.bfloat16),    # ragged last tile, one round per wave
    (8, 1000, 768, 16, torch.float16),     # three rounds: one wave idle
    (16, 777, 2048, 32, torch.bfloat16),   # one round pair per wave
    (16, 64, 5120, 64, torch.bfloat16),    # five rounds per wave: pairs and a tail round
    (12, 4096, 14336, 8, torch.bfloat16),  # down-projection shape
    (2, 300, 256, 32, torch.float16),      # M <= 4 with K % 1024 != 0; a single round
    (16, 16, 256, 8, torch.float16),
    (9, 4096, 4096, 32, torch.bfloat16),
])
def test_e8b_gemv16_kernel_matches_oracle(M, N, K, gs, dtype):
    # M <= 16 (above 4, or K % 1024 != 0), K % 256 == 0 and gs in {8, 16, 32, 64} select
    # the 2-bit GEMV with the weights in the B operand
    pk, sc, pk_np, sc_np = _layer2(N, K, seed=3 * N + K + gs, gs=gs)
    g = torch.Generator().manual_seed(M * 7 + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"e8b gemv16 M={M} N={N} K={K} gs={gs} {dtype}", flush=True)
    y = ops.e8_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, gs)
    y_nb = ops.e8_linear(x.to(DEV), pk, sc, None, N, K, gs)
    torch.cuda.synchronize()
    ref = O.e8b_gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, gs,
                         DT_CODE[dtype])
    ref_nb = O.e8b_gemm_f64(x.float().numpy(), pk_np, sc_np, None, N, K, gs, DT_CODE[dtype])
    assert y.shape == (M, N) and y.dtype == dtype
    assert _rel_err(y, ref) <= REL_TOL
    assert _rel_err(y_nb, ref_nb) <= REL_TOL


@pytest.mark.parametrize("M,N,K,gs,dtype", [
    (17, 256, 512, 8, torch.bfloat16),
    (100, 1000, 256, 16, torch.float16),
    (256, 256, 1024, 32, torch.bfloat16),
    (300, 520, 512, 64, torch.float16),
    (513, 96, 128, 8, torch.bfloat16),
    (64, 4096, 64, 32, torch.bfloat16),
    (40, 1024, 4096, 8, torch.bfloat16),   # small grid: K split over 16 steps per split
    (201, 301, 1344, 16, torch.float16),   # 21 K steps over uneven splits, ragged M and N
    (20, 2048, 2048, 64, torch.float16),   # small batch just above the GEMV range
])
def test_e8b_prefill_mfma_matches_oracle(M, N, K, gs, dtype):
    # K % 64 == 0, gs in {8, 16, 32, 64} and M > 16 (or K % 256 != 0) select the MFMA GEMM
    # with the 2-bit weight decoder
    pk, sc, pk_np, sc_np = _layer2(N, K, seed=M + N + K + gs, gs=gs)
    g = torch.Generator().manual_seed(M * 3 + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"e8b prefill M={M} N={N} K={K} gs={gs} {dtype}", flush=True)
    y = ops.e8_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, gs)
    torch.cuda.synchronize()
    ref = O.e8b_gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, gs,
                         DT_CODE[dtype])
    assert y.shape == (M, N) and y.dtype == dtype
    assert _rel_err(y, ref) <= REL_TOL


@pytest.mark.parametrize("gs", [8, 32])
@pytest.mark.parametrize("M,name,N,K", [(512, "gate_up", 14336, 4096), (2048, "down", 4096, 14336),
                                        (512, "q_o", 4096, 4096)])
def test_e8b_prefill_llama8b_shapes(M, name, N, K, gs):
    # every element against an fp32 matmul of the decoded weights (the decoder is pinned
    # bit-exact above), plus a row sample against the fp64 oracle
    gw = torch.Generator(device=DEV).manual_seed(9100 + N + gs)
    w = torch.randn(N, K, generator=gw, device=DEV) * 0.02
    pk, sc = ops.encode2(w, gs)
    del w
    x = torch.randn(M, K, generator=gw, device=DEV).to(torch.bfloat16)
    print(f"e8b prefill {name} M={M} gs={gs}", flush=True)
    y = ops.e8_linear(x, pk, sc, None, N, K, gs)
    wdq = ops.decode2(pk, sc, N * K, gs, torch.bfloat16).view(N, K).float()
    ref = x.float() @ wdq.t().contiguous()
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    err = ((y.float() - ref).abs().max() / ref.abs().max()).item()
    assert err <= REL_TOL
    rows = [0, 1, 255, 256, M - 1]
    ref64 = O.e8b_gemm_f64(x[rows].float().cpu().numpy(), pk.cpu().numpy(), _u16(sc), None, N, K,
                           gs, O.DT_BF16)
    assert _rel_err(y[rows], ref64) <= REL_TOL
