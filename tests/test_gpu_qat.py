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
    with pytest.raises(RuntimeError, match="float32 and float64"):
        ojasx_amd.conway_sloane_e8_project(torch.zeros(2, 8, device=DEV, dtype=torch.float16))


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
