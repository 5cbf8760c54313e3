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


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(201, 301, 1344), (40, 1024, 8192), (129, 640, 2048)])
def test_prefill_k_split_uneven_steps_and_ragged_tail(dtype, M, N, K):
    # small grids run split over K: 21 K steps over 2 splits (uneven), 128 steps over the
    # maximum of 16 splits, and M*N not a multiple of 4 (the reduction's scalar tail)
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=M * 3 + N + K)
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    print(f"prefill split M={M} N={N} K={K} {dtype}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32,
                     DT_CODE[dtype])
    assert _rel(y, ref) <= REL_TOL


def test_prefill_k_split_scratch_growth_and_reuse():
    # the K-split scratch grows with the request and is reused by smaller ones afterwards
    cases = [(64, 256, 1024), (512, 1024, 4096), (96, 512, 2048), (600, 2048, 4096),
             (64, 256, 1024)]
    for i, (M, N, K) in enumerate(cases):
        pk, sc, pk_np, sc_np = _encoded(N, K, seed=40 + i)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(i)).to(torch.bfloat16)
        print(f"prefill scratch case {i} M={M} N={N} K={K}", flush=True)
        y = ops.e8t_linear(x.to(DEV), pk, sc, None, N, K, 32)
        torch.cuda.synchronize()
        rows = list(range(0, M, max(1, M // 16))) + [M - 1]
        ref = O.gemm_f64(x[rows].float().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
        assert _rel(y[rows], ref) <= REL_TOL


def test_prefill_graph_capture_keeps_split_and_matches_eager():
    # the K-split workspace comes from torch's allocator, so the captured launch keeps the
    # split (its workspace lives in the graph's pool); every replay (with eager split work
    # in between) is bit-identical to the eager result
    M, N, K = 512, 1024, 4096
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=77)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV)
    y_eager = ops.e8t_linear(x, pk, sc, None, N, K, 32)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.e8t_linear(x, pk, sc, None, N, K, 32)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_graph = ops.e8t_linear(x, pk, sc, None, N, K, 32)
    rows = [0, 1, 255, 511]
    ref = O.gemm_f64(x[rows].float().cpu().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
    assert _rel(y_eager[rows], ref) <= REL_TOL
    for rep in range(3):
        y_graph.fill_(float("nan"))
        ops.e8t_linear(x, pk, sc, None, N, K, 32)  # eager (split) work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert _rel(y_graph[rows], ref) <= REL_TOL, rep
        assert torch.equal(y_graph, y_eager), rep


def test_prefill_large_tile_k_split_uneven_and_ragged():
    # 4 x 24 large tiles split 3 ways over 65 K steps (21/22/22), ragged M and N, bias
    M, N, K = 1000, 6100, 4160
    gw = torch.Generator(device=DEV).manual_seed(4242)
    w = torch.randn(N, K, generator=gw, device=DEV) * 0.02
    pk, sc = ops.encode(w, 32)
    del w
    x = torch.randn(M, K, generator=gw, device=DEV).to(torch.bfloat16)
    bias = torch.randn(N, generator=gw, device=DEV).to(torch.bfloat16)
    print(f"prefill large split M={M} N={N} K={K}", flush=True)
    y = ops.e8t_linear(x, pk, sc, bias, N, K, 32)
    wdq = ops.decode(pk, sc, N * K, 32, torch.bfloat16).view(N, K).float()
    ref = x.float() @ wdq.t().contiguous() + bias.float()
    torch.cuda.synchronize()
    assert _rel(y, ref) <= REL_TOL
    rows = [0, 255, 256, 511, 999]
    ref64 = O.gemm_f64(x[rows].float().cpu().numpy(), pk.cpu().numpy(),
                       sc.cpu().view(torch.int16).numpy().view(np.uint16),
                       bias.float().cpu().numpy(), N, K, 32, O.DT_BF16)
    assert _rel(y[rows], ref64) <= REL_TOL
