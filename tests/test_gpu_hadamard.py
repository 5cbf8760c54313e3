"""GPU parity of the HIP fwht_block32 kernel (ojx_fwht32 / ops.fwht32).

The reference's fwht_block32 (ojasx2/math/lattice.py:91-102) is five torch stages of
butterflies plus one multiply by 0.1767766952966369.  The kernel must reproduce it bit for
bit: the expected values are torch's own evaluation of the stages on the CPU (each stage
rounded to the tensor's dtype by torch), for fp32, fp16, bf16 and fp64.  Independently, the
result is the normalised Sylvester-Hadamard matrix applied to each 32-block (fp64, scipy's
matrix) and the transform is an involution.  The fused linear with use_hadamard runs it on x
and on grad_x (lattice.py:564-565, 713-714); its layer tests live in test_gpu_linear.py.
"""

import math

import numpy as np
import pytest
import torch
from scipy.linalg import hadamard

import ojasx_amd
from ojasx_amd import _native as N
from ojasx_amd import ops

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _stages_cpu(x):
    # distance d: element i (bit d clear) <- x_i + x_{i+d}, element i + d <- x_i - x_{i+d}
    h = x.reshape(-1, 32).clone()
    for d in (1, 2, 4, 8, 16):
        out = h.clone()
        for i in range(32):
            if (i // d) % 2 == 0:
                out[:, i] = h[:, i] + h[:, i + d]
                out[:, i + d] = h[:, i] - h[:, i + d]
        h = out
    return (h * 0.1767766952966369).reshape(x.shape)


def _bits(t):
    if t.dtype == torch.float64:
        return t.view(torch.int64)
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    return t.view(torch.int16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("shape", [(1, 32), (3, 5, 96), (257, 64), (4096,)])
def test_fwht32_bit_exact_to_torch_stages(dtype, shape):
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(*shape, generator=g, dtype=torch.float64)
    x = x * torch.exp2(torch.randint(-12, 12, shape, generator=g).double())  # wide exponents
    x = x.to(dtype)
    print(f"fwht32 {dtype} {shape}", flush=True)
    y = ops.fwht32(x.to(DEV))
    torch.cuda.synchronize()
    ref = _stages_cpu(x)
    assert y.dtype == dtype and y.shape == x.shape
    assert torch.equal(_bits(y.cpu()), _bits(ref))


def test_fwht32_is_the_normalised_hadamard_matrix_and_an_involution():
    x = torch.randn(64, 128, dtype=torch.float64)
    H = torch.from_numpy(hadamard(32).astype(np.float64)) / math.sqrt(32)
    y = ops.fwht32(x.to(DEV)).cpu()
    assert torch.allclose(y, (x.view(64, 4, 32) @ H.T).view(64, 128), atol=1e-13)
    assert torch.allclose(ops.fwht32(y.to(DEV)).cpu(), x, atol=1e-13)
    xf = torch.randn(16, 64)
    assert torch.allclose(ops.fwht32(ops.fwht32(xf.to(DEV))).cpu(), xf, atol=1e-5)


def test_fwht_block32_routes_gpu_tensors_and_keeps_reference_rules():
    x = torch.randn(6, 64, device=DEV).to(torch.bfloat16)
    assert torch.equal(ojasx_amd.fwht_block32(x).cpu(), _stages_cpu(x.cpu()))
    view = torch.randn(64, 96, device=DEV)[:, 32:]  # non-contiguous rows
    assert torch.equal(ojasx_amd.fwht_block32(view).cpu(), _stages_cpu(view.cpu()))
    odd = torch.randn(3, 30, device=DEV)
    assert ojasx_amd.fwht_block32(odd) is odd  # not a multiple of 32: unchanged


def test_fwht32_gradient_is_the_transform():
    x = torch.randn(8, 64, device=DEV, dtype=torch.float64, requires_grad=True)
    gy = torch.randn(8, 64, device=DEV, dtype=torch.float64)
    ojasx_amd.fwht_block32(x).backward(gy)
    H = torch.from_numpy(hadamard(32).astype(np.float64)).to(DEV) / math.sqrt(32)
    assert torch.allclose(x.grad, (gy.view(8, 2, 32) @ H).view(8, 64), atol=1e-13)


def test_fwht32_c_abi_rejects_bad_layouts():
    L = N.lib()
    x = torch.zeros(64, device=DEV)
    assert L.ojx_fwht32(x.data_ptr(), 0, 48, x.data_ptr(), 0) != 0
    assert b"multiple of 32" in L.ojx_e8t_last_error()
    assert L.ojx_fwht32(x.data_ptr() + 4, 0, 32, x.data_ptr(), 0) != 0
    assert L.ojx_fwht32(x.data_ptr(), 7, 32, x.data_ptr(), 0) != 0
    assert L.ojx_fwht32(x.data_ptr(), 0, 0, x.data_ptr(), 0) == 0
    # in place
    y = torch.randn(4, 32, device=DEV)
    ref = _stages_cpu(y.cpu())
    assert L.ojx_fwht32(y.data_ptr(), 0, y.numel(), y.data_ptr(),
                        N.stream_handle(DEV)) == 0
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), ref)
