"""GPU parity of the prefill MFMA GEMM (batch M > 16).

Bar (north star): max|y - y_ref| / max|y_ref| <= 1e-2 with fp32/fp64 accumulation in
the reference, the weights following the reference's dtype rule (coord *
scales.to(dtype), lattice.py:414-418).

* small and ragged shapes: every element against the fp64 CPU oracle;
* BASELINE configs[2] shapes (Llama-3-8B linears, M = 512 and 2048): every element
  against an fp32 GPU matmul of the decoded weights (the decoder is pinned bit-exact
  to the oracle by test_gpu_codec.py), plus a row sample against the fp64 oracle.
"""

import numpy as np
import pytest
import torch

from ojasx_amd import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
REL_TOL = 1e-2
DT_CODE = {torch.float16: O.DT_F16, torch.bfloat16: O.DT_BF16}


def _encoded(N, K, seed, scale=0.02):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * scale
    packed, s16, _ = O.encode(w.numpy(), 32)
    return (torch.from_numpy(packed).to(DEV), torch.from_numpy(s16.view(np.float16).copy()).to(DEV),
            packed, s16)


def _rel(y, ref):
    y = y.detach().float().cpu().numpy() if isinstance(y, torch.Tensor) else y
    ref = ref.detach().double().cpu().numpy() if isinstance(ref, torch.Tensor) else ref
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(17, 256, 512), (100, 1000, 256), (256, 256, 1024),
                                   (300, 520, 512), (513, 96, 128), (64, 4096, 64)])
def test_prefill_matches_oracle(dtype, M, N, K):
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=M + N + K)
    g = torch.Generator().manual_seed(K)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"prefill M={M} N={N} K={K} {dtype}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32,
                     DT_CODE[dtype])
    assert y.shape == (M, N) and y.dtype == dtype
    assert _rel(y, ref) <= REL_TOL


@pytest.mark.parametrize("M", [512, 2048])
@pytest.mark.parametrize("name,N,K", [("q_o", 4096, 4096), ("k_v", 1024, 4096),
                                      ("gate_up", 14336, 4096), ("down", 4096, 14336)])
def test_prefill_llama8b_shapes_full(name, N, K, M):
    sid = ["q_o", "k_v", "gate_up", "down"].index(name)
    gw = torch.Generator(device=DEV).manual_seed(8200 + sid)
    w = torch.randn(N, K, generator=gw, device=DEV) * 0.02
    pk, sc = ops.encode(w, 32)
    del w
    gx = torch.Generator(device=DEV).manual_seed(8400 + M)
    x = torch.randn(M, K, generator=gx, device=DEV).to(torch.bfloat16)
    print(f"prefill {name} M={M}", flush=True)
    y = ops.e8t_linear(x, pk, sc, None, N, K, 32)
    wdq = ops.decode(pk, sc, N * K, 32, torch.bfloat16).view(N, K).float()
    ref = x.float() @ wdq.t().contiguous()
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert _rel(y, ref) <= REL_TOL
    rows = [0, 1, 127, 128, 255, 256, M - 1]
    ref64 = O.gemm_f64(x[rows].float().cpu().numpy(), pk.cpu().numpy(),
                       sc.cpu().view(torch.int16).numpy().view(np.uint16), None, N, K, 32,
                       O.DT_BF16)
    assert _rel(y[rows], ref64) <= REL_TOL


def test_prefill_unaligned_input_falls_back():
    N, K, M = 128, 256, 40
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=2)
    xb = torch.randn(M * K + 1, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    x = xb.to(DEV)[1:].view(M, K)  # not 16-byte aligned: general kernel
    y = ops.e8t_linear(x, pk, sc, None, N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().cpu().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
    assert _rel(y, ref) <= REL_TOL
