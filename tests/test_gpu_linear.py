"""GPU parity of the fused E8 linear (forward, backward dX) and of the layer API.

Bar (north star): matmul outputs within max relative error 1e-2 of the fp64
dequantize-then-matmul oracle for bf16/fp16 activations, measured as
max|y - y_ref| / max|y_ref|; fp32 activations within abs 1e-4 at the reference
test's small shapes (tests/test_fused_e8_gemm.py:129-182 of the reference)."""

import concurrent.futures as cf

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
REL_TOL = 1e-2   # bf16 / fp16 activations (north star)
ABS_TOL_F32 = 1e-4


def _layer(N, K, seed, gs=32, scale=0.02):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * scale
    packed, s16, _ = O.encode(w.numpy(), gs)
    return (torch.from_numpy(packed).to(DEV),
            torch.from_numpy(s16.view(np.float16).copy()).to(DEV), packed, s16)


def _rel_err(y: torch.Tensor, ref: np.ndarray) -> float:
    return float(np.abs(y.detach().float().cpu().numpy() - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(1, 256, 512), (3, 128, 256), (16, 96, 1024),
                                   (64, 192, 512), (130, 64, 256), (5, 40, 96)])
def test_fwd_matches_oracle(dtype, M, N, K):
    pk, sc, pk_np, sc_np = _layer(N, K, seed=M * 131 + N)
    g = torch.Generator().manual_seed(K)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32, DT_CODE[dtype])
    assert y.dtype == dtype and y.shape == (M, N)
    if dtype == torch.float32:
        assert float(np.abs(y.cpu().numpy() - ref).max()) <= ABS_TOL_F32
    else:
        assert _rel_err(y, ref) <= REL_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(1, 256, 512), (7, 96, 256), (33, 64, 128)])
def test_bwd_dx_matches_oracle(dtype, M, N, K):
    pk, sc, pk_np, sc_np = _layer(N, K, seed=N + K)
    gy = torch.randn(M, N).to(dtype)
    gx = ops.e8t_linear_bwd_dx(gy.to(DEV), pk, sc, N, K, 32)
    ref = O.gemm_bwd_f64(gy.float().numpy(), pk_np, sc_np, N, K, 32, DT_CODE[dtype])
    if dtype == torch.float32:
        assert float(np.abs(gx.cpu().numpy() - ref).max()) <= ABS_TOL_F32
    else:
        assert _rel_err(gx, ref) <= REL_TOL


@pytest.mark.parametrize("name,N,K", [("q_o", 4096, 4096), ("k_v", 1024, 4096),
                                      ("gate_up", 14336, 4096), ("down", 4096, 14336)])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_decode_gemv_llama8b_shapes(name, N, K, M):
    # BASELINE C2: W ~ N(0, 0.02) from seed 8200 + shape id, x bf16 N(0,1) seed 8300 + M
    sid = ["q_o", "k_v", "gate_up", "down"].index(name)
    pk, sc, pk_np, sc_np = _layer(N, K, seed=8200 + sid)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(8300 + M)).to(torch.bfloat16)
    y = ops.e8t_linear(x.to(DEV), pk, sc, None, N, K, 32)
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
    assert _rel_err(y, ref) <= REL_TOL


@pytest.mark.parametrize("name,N,K", [("q_o", 4096, 4096), ("k_v", 1024, 4096),
                                      ("gate_up", 14336, 4096), ("down", 4096, 14336)])
def test_prefill_llama8b_shapes_row_sample(name, N, K):
    # BASELINE C3 at M = 512: the full product is checked on a row sample of x
    # (rows are independent), the rest through the finite / shape contract.
    M = 512
    sid = ["q_o", "k_v", "gate_up", "down"].index(name)
    pk, sc, pk_np, sc_np = _layer(N, K, seed=8200 + sid)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(8400 + M)).to(torch.bfloat16)
    y = ops.e8t_linear(x.to(DEV), pk, sc, None, N, K, 32)
    assert torch.isfinite(y).all()
    rows = [0, 1, 255, 511]
    ref = O.gemm_f64(x[rows].float().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
    assert _rel_err(y[rows], ref) <= REL_TOL


def test_fused_ternary_gemm_parity_reference_test():
    # reference tests/test_fused_e8_gemm.py:129-150 on the device path (fp32, abs 1e-4)
    torch.manual_seed(42)
    ref_linear = nn.Linear(128, 256, bias=True).to(DEV)
    layer = ojasx_amd.E8LatticeLinear.from_linear(ref_linear, rank=4, bitrate=1.5, group_size=32)
    x = torch.randn(3, 8, 128, device=DEV)
    w_unpacked = layer.unpack_weights(dtype=x.dtype)
    expected = F.linear(x, w_unpacked, layer.bias)
    expected = expected + layer.scaling * ((x @ layer.lora_A) @ layer.lora_B)
    out = layer.forward_fused(x)
    assert float((out - expected).detach().abs().max()) < 1e-4


def test_native_schema_ops_match_layer():
    # torch.ops.ojasx_e8t.fused_ternary_e8_gemm_fwd keeps the reference native schema
    torch.manual_seed(99)
    ref_linear = nn.Linear(64, 128, bias=True).to(DEV)
    layer = ojasx_amd.E8LatticeLinear.from_linear(ref_linear, rank=0, bitrate=1.5, group_size=32)
    x = torch.randn(2, 64, device=DEV)
    packed_2d = layer.packed_weight.reshape(128, 64 * 3 // 16)
    scales_2d = layer.block_scales.reshape(128, -1)
    y = torch.ops.ojasx_e8t.fused_ternary_e8_gemm_fwd(x, packed_2d, scales_2d, layer.bias, 32)
    exp = F.linear(x, layer.unpack_weights(dtype=x.dtype), layer.bias)
    assert float((y - exp).detach().abs().max()) < 1e-4
    gy = torch.randn(2, 128, device=DEV)
    gx = torch.ops.ojasx_e8t.fused_ternary_e8_gemm_bwd_dx(gy, packed_2d, scales_2d, 64, 32)
    assert float((gx - gy @ layer.unpack_weights()).detach().abs().max()) < 1e-4
    with pytest.raises(RuntimeError, match="divisible"):
        torch.ops.ojasx_e8t.fused_ternary_e8_gemm_fwd(torch.randn(2, 30, device=DEV), packed_2d,
                                                      scales_2d, None, 32)


def test_layer_forward_backward_lora_grads():
    # reference tests/test_sub2bit_lattice.py:65-94
    torch.manual_seed(77)
    linear = nn.Linear(256, 512, bias=True).to(DEV)
    layer = ojasx_amd.E8LatticeLinear.from_linear(linear, rank=8, bitrate=1.5, group_size=32)
    assert layer.packed_weight.numel() == int(256 * 512 * 1.5 / 8)
    x = torch.randn(2, 4, 256, device=DEV, requires_grad=True)
    out = layer(x)
    assert out.shape == (2, 4, 512) and torch.isfinite(out).all()
    out.sum().backward()
    assert layer.lora_A.grad is not None and layer.lora_B.grad is not None
    assert not layer.packed_weight.requires_grad and not layer.block_scales.requires_grad
    # dX against unpack + matmul
    w = layer.unpack_weights()
    gx_ref = torch.ones(2, 4, 512, device=DEV) @ w
    gx_ref = gx_ref + layer.scaling * (torch.ones(2, 4, 512, device=DEV) @ layer.lora_B.t() @ layer.lora_A.t())
    assert float((x.grad - gx_ref).detach().abs().max()) < 1e-3


def test_layer_default_group_size_coerced():
    # reference tests/test_sub2bit_lattice.py:97-108
    layer = ojasx_amd.E8LatticeLinear.from_linear(nn.Linear(64, 64).to(DEV), bitrate=1.5)
    assert layer.group_size == 16
    assert layer.block_scales.shape[0] == (64 * 64) // 16
    out = layer(torch.randn(2, 64, device=DEV))
    assert out.shape == (2, 64) and torch.isfinite(out).all()


@pytest.mark.parametrize("shape", [(16, 32), (7, 13), (5, 19)])
def test_arbitrary_shapes_with_hadamard(shape):
    # reference tests/test_ojasx_exhaustive.py:299-320 (ternary row)
    torch.manual_seed(77)
    out_f, in_f = shape
    lin = nn.Linear(in_f, out_f, bias=True).to(DEV)
    e8 = ojasx_amd.E8LatticeLinear.from_linear(lin, rank=4, bitrate=1.5,
                                               use_hadamard=(in_f % 32 == 0))
    w = e8.unpack_weights()
    assert w.shape == (out_f, in_f) and torch.isfinite(w).all()
    x = torch.randn(3, in_f, device=DEV, requires_grad=True)
    y = e8(x)
    assert y.shape == (3, out_f)
    # the forward equals unpack + linear (+ LoRA) including the Hadamard pair
    exp = F.linear(x, w, e8.bias) + e8.scaling * ((x @ e8.lora_A) @ e8.lora_B)
    assert float((y - exp).detach().abs().max()) < 1e-4
    y.sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    assert e8.lora_A.grad is not None and e8.lora_B.grad is not None


def test_pack_model_e8_targets_and_excludes():
    model = nn.Sequential(nn.Linear(64, 128), nn.ReLU(),
                          nn.Sequential(nn.Linear(128, 64), nn.Linear(64, 32))).to(DEV)
    packed = ojasx_amd.pack_model_e8(model, rank=2, group_size=32, bitrate=1.5,
                                     exclude_modules=["0"], inplace=False)
    assert isinstance(packed[0], nn.Linear)  # excluded by name "0"
    assert isinstance(packed[2][1], ojasx_amd.E8LatticeLinear)
    x = torch.randn(4, 64, device=DEV)
    assert packed(x).shape == (4, 32)


def test_concurrent_threads_share_no_state():
    # reference tests/test_ojasx_exhaustive.py:323-345
    layers = [ojasx_amd.E8LatticeLinear.from_linear(nn.Linear(64, 64).to(DEV), bitrate=1.5,
                                                    group_size=32) for _ in range(4)]
    inputs = [torch.randn(8, 64, device=DEV) for _ in range(4)]
    expected = [layers[i](inputs[i]) for i in range(4)]

    def work(i):
        with torch.cuda.stream(torch.cuda.Stream()):
            for _ in range(10):
                out = layers[i](inputs[i])
            torch.cuda.current_stream().synchronize()
        return out

    with cf.ThreadPoolExecutor(max_workers=4) as pool:
        results = list(pool.map(work, range(4)))
    for i in range(4):
        assert torch.equal(results[i], expected[i])


def test_empty_batch_and_zero_rows():
    pk, sc, _, _ = _layer(64, 128, seed=1)
    y = ops.e8t_linear(torch.empty(0, 128, device=DEV, dtype=torch.bfloat16), pk, sc, None, 64, 128, 32)
    assert y.shape == (0, 64)


def test_bad_layouts_raise():
    pk, sc, _, _ = _layer(64, 128, seed=1)
    with pytest.raises(RuntimeError, match="features"):
        ops.e8t_linear(torch.randn(2, 64, device=DEV), pk, sc, None, 64, 128, 32)
    with pytest.raises(RuntimeError, match="needs"):
        ops.e8t_linear(torch.randn(2, 256, device=DEV), pk, sc, None, 64, 256, 32)
    with pytest.raises(RuntimeError, match="float32, float16 and bfloat16"):
        ops.e8t_linear(torch.randn(2, 128, device=DEV, dtype=torch.float64), pk, sc, None, 64, 128, 32)
