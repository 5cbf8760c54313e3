"""GPU parity of the Conway-Sloane E8 projection and the QAT straight-through quantizer
(ojasx2/math/lattice.py:162-203, 853-898): bit-exact with the CPU oracle, which is pinned
bit for bit to torch's evaluation of the reference's expressions (tests/test_oracle_qat.py)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import ojasx_amd
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _inputs(dtype, n=100_000, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, 8, generator=g) * 3).to(dtype)
    x[:2000] = torch.round(x[:2000] * 2) / 2
    x[2000:3000] = torch.round(x[2000:3000])
    x[3000:3100] = 0.0
    x[3100:3200] = -0.0
    x[3200:3300, :] = 0.5
    return x


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_cs_project_bit_exact(dtype):
    x = _inputs(dtype)
    print(f"cs_project {dtype}", flush=True)
    got = ojasx_amd.conway_sloane_e8_project(x.to(DEV))
    torch.cuda.synchronize()
    assert got.dtype == dtype and got.shape == x.shape
    assert np.array_equal(got.cpu().numpy(), O.cs_project(x.numpy()))
    # CPU tensors come back on the CPU; other shapes keep their shape
    y = ojasx_amd.conway_sloane_e8_project(x[:64].view(4, 2, 8, 8))
    assert y.device.type == "cpu" and y.shape == (4, 2, 8, 8)
    assert np.array_equal(y.reshape(-1, 8).numpy(), O.cs_project(x[:64].numpy()))


def test_cs_project_errors_and_empty():
    with pytest.raises(ValueError, match="Last dimension must be 8"):
        ojasx_amd.conway_sloane_e8_project(torch.zeros(3, 7, device=DEV))
    e = torch.zeros(0, 8, device=DEV)
    assert ojasx_amd.conway_sloane_e8_project(e).shape == (0, 8)
    with pytest.raises(RuntimeError, match="float32, float64, float16 and bfloat16"):
        ojasx_amd.conway_sloane_e8_project(torch.zeros(2, 8, device=DEV, dtype=torch.int32))


@pytest.mark.parametrize("shape", [(1000, 37), (4096, 4096), (3, 5), (1, 1)])
def test_ste_quantize_bit_exact(shape):
    g = torch.Generator().manual_seed(sum(shape))
    w = torch.randn(*shape, generator=g) * 0.05
    w.view(-1)[: min(4, w.numel())] = 0.0
    print(f"ste_quantize {shape}", flush=True)
    got = ojasx_amd._E8STEFunction.apply(w.to(DEV))
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), O.ste_quantize(w.numpy()))


def test_qat_linear_forward_uses_quantized_weight_and_straight_through_grad():
    torch.manual_seed(3)
    layer = ojasx_amd.E8QuantizationAwareLinear(64, 32).to(DEV)
    x = torch.randn(5, 64, device=DEV, requires_grad=True)
    y = layer(x)
    w_q = torch.from_numpy(O.ste_quantize(layer.weight.detach().cpu().numpy())).to(DEV)
    assert torch.allclose(y, F.linear(x, w_q, layer.bias), atol=1e-5, rtol=1e-5)
    y.square().sum().backward()
    gy = 2 * y.detach()
    # straight through: dL/dW = gy^T x, as for an unquantized linear
    assert torch.allclose(layer.weight.grad, gy.t() @ x.detach(), atol=1e-4, rtol=1e-4)
    assert torch.allclose(x.grad, gy @ w_q, atol=1e-4, rtol=1e-4)


def _half_inputs(dtype, n=100_000, seed=7):
    x = _inputs(torch.float32, n, seed)
    g = torch.Generator().manual_seed(seed + 1)
    # magnitudes where the half type rounds x - 0.5, f +- 1 and the parity sum
    x[4000:6000] = torch.randn(2000, 8, generator=g) * 400
    x[6000:7000] = torch.round(torch.randn(1000, 8, generator=g) * 300)
    x[7000:7100] = torch.tensor([256.0, 1, 1, 1, 1, 1, 1, 1])
    x[7100:7200] = torch.tensor([2048.0, 1, 1, 1, 1, 1, 1, 0.5])
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_cs_project_half_bit_exact(dtype):
    # the reference's projection on an fp16 / bf16 tensor rounds every op to the dtype
    # (lattice.py:180-203); bit for bit against the oracle pinned to torch's evaluation
    x = _half_inputs(dtype)
    print(f"cs_project {dtype}", flush=True)
    got = ojasx_amd.conway_sloane_e8_project(x.to(DEV))
    torch.cuda.synchronize()
    assert got.dtype == dtype and got.shape == x.shape
    ref = O.cs_project_half(x.float().numpy(), dtype == torch.bfloat16)
    assert np.array_equal(got.float().cpu().numpy(), ref, equal_nan=True)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1000, 37), (4096, 4096), (3, 5), (1, 1)])
def test_ste_quantize_half_bit_exact(dtype, shape):
    g = torch.Generator().manual_seed(sum(shape) + 11)
    w = (torch.randn(*shape, generator=g) * 0.05).to(dtype)
    w.view(-1)[: min(4, w.numel())] = 0.0
    if w.numel() >= 32:
        w.view(-1)[8:16] = 0.0          # zero 8-vector (fp16: s = 0, NaN outputs)
        w.view(-1)[16:24] = 3e-5
    print(f"ste_quantize {dtype} {shape}", flush=True)
    got = ojasx_amd._E8STEFunction.apply(w.to(DEV))
    torch.cuda.synchronize()
    assert got.dtype == dtype
    ref = O.ste_quantize_half(w.float().numpy(), dtype == torch.bfloat16)
    assert np.array_equal(got.float().cpu().numpy().reshape(-1), ref.reshape(-1), equal_nan=True)


def test_qat_linear_bf16_forward_and_backward():
    # E8QuantizationAwareLinear(dtype=bfloat16): the quantizer runs in bf16, the linear in
    # bf16, the gradient passes straight through
    torch.manual_seed(5)
    layer = ojasx_amd.E8QuantizationAwareLinear(64, 32, device=DEV, dtype=torch.bfloat16)
    x = torch.randn(5, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    y = layer(x)
    assert y.dtype == torch.bfloat16
    w_q = torch.from_numpy(O.ste_quantize_half(layer.weight.detach().float().cpu().numpy(),
                                               True)).to(DEV).to(torch.bfloat16)
    ref = F.linear(x.detach().float(), w_q.float(), layer.bias.detach().float())
    assert float((y.detach().float() - ref).abs().max() / ref.abs().max()) <= 1e-2
    y.float().square().sum().backward()
    gy = (2 * y.detach().float())
    assert torch.allclose(layer.weight.grad.float(), gy.t() @ x.detach().float(), rtol=2e-2,
                          atol=2e-2 * float((gy.t() @ x.detach().float()).abs().max()))
    assert torch.allclose(x.grad.float(), gy @ w_q.float(), rtol=2e-2,
                          atol=2e-2 * float((gy @ w_q.float()).abs().max()))
