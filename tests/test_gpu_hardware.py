"""GPU runs of the ``ojasx3.hardware`` entry's packed-weight call
(UniversalCompiledKernel.__call__, tilelang_kernels.py:497-549).

* the reference's own parity case (tests/test_emitted_cpu_kernel.py:177-182): an
  E8LatticeLinear's packed buffers through the kernel object against
  ``F.linear(x, unpack_weights(), bias)``, fp32 at rtol = atol = 1e-4, for each bitrate;
* routing: bf16 and leading batch dims give exactly the bits of the format's own op
  (the same HIP kernels), and the result is within 1e-2 of the fp64 oracle.
"""

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from ojasx_amd import hardware as H
from ojasx_amd import ops
from ojasx_amd.lattice import E8LatticeLinear

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("bitrate", [2.0, 1.5, 1.0])
def test_packed_call_matches_unpack_linear_fp32(bitrate):
    torch.manual_seed(7)
    M, N, K = 32, 64, 64
    print(f"hardware entry fp32 bitrate={bitrate}", flush=True)
    kernel = H.compile_or_emit_universal_kernel(M, N, K, device="cuda", bitrate=bitrate,
                                                group_size=32, dtype=torch.float32)
    x = torch.randn(M, K, device=DEV)
    layer = E8LatticeLinear.from_linear(nn.Linear(K, N, bias=True).to(DEV), rank=0,
                                        bitrate=bitrate, group_size=32)
    out = kernel(x, layer.packed_weight, layer.block_scales, layer.bias)
    expected = F.linear(x, layer.unpack_weights(dtype=x.dtype), layer.bias)
    torch.cuda.synchronize()
    torch.testing.assert_close(out, expected, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(kernel(x, layer), layer.forward_fused(x), rtol=0, atol=0)


@pytest.mark.parametrize("bitrate,gs", [(1.5, 32), (2.0, 8), (1.0, 32)])
@pytest.mark.parametrize("M", [1, 40])
def test_packed_call_routes_to_format_op(bitrate, gs, M):
    N, K = 256, 1024
    g = torch.Generator().manual_seed(int(bitrate * 10) + M)
    w = (torch.randn(N, K, generator=g) * 0.02).to(DEV)
    enc, lin = {1.5: (ops.encode, ops.e8t_linear), 2.0: (ops.encode2, ops.e8_linear),
                1.0: (ops.encode1, ops.e8r_linear)}[bitrate]
    packed, scales = enc(w, gs)
    x = torch.randn(2, M, K, generator=g).to(torch.bfloat16).to(DEV)
    bias = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV)
    print(f"hardware entry routing bitrate={bitrate} gs={gs} M={M}", flush=True)
    kernel = H.compile_or_emit_universal_kernel(2 * M, N, K, bitrate=bitrate, group_size=gs,
                                                dtype=torch.bfloat16)
    y = kernel(x, packed, scales, bias)
    y_op = lin(x, packed, scales, bias, N, K, gs)
    torch.cuda.synchronize()
    assert y.shape == (2, M, N) and torch.equal(y, y_op)
    wdq = {1.5: ops.decode, 2.0: ops.decode2, 1.0: ops.decode1}[bitrate](
        packed, scales, N * K, gs, torch.bfloat16).view(N, K)
    ref = (x.double().reshape(-1, K) @ wdq.double().t() + bias.double()).cpu().numpy()
    err = np.abs(y.reshape(-1, N).double().cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 1e-2
