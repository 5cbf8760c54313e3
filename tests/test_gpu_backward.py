"""GPU parity of the MFMA backward dX (grad_x = grad_y . Wdeq) for the three formats.

Bar: max|gx - ref| / max|ref| <= 1e-2 for bf16 / fp16 against the fp64 oracle (the
reference's backward, lattice.py:684-717; native fused_*_gemm_bwd_dx), with the weights
under each format's dtype rule.  Shapes with N % 64 == 0 and K % 64 == 0 run the MFMA
kernel (transposed weight tiles); ragged M and output widths that are not a multiple of
the tile, and reductions split over N, are covered; Llama-3-8B shapes are checked on every
element against an fp32 matmul of the bit-exact decoded weights."""

import numpy as np
import pytest
import torch

from ojasx_amd import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
REL_TOL = 1e-2
DT_CODE = {torch.float16: O.DT_F16, torch.bfloat16: O.DT_BF16}
SHAPES = [(17, 256, 512), (100, 1024, 256), (300, 128, 640), (513, 64, 128),
          (40, 4096, 1024), (3, 192, 320)]


def _rel(y, ref):
    y = y.detach().float().cpu().numpy()
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _w(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * 0.02).numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_ternary_bwd_mfma(dtype, M, N, K):
    pk, s16, _ = O.encode(_w(N, K, M + N), 32)
    gy = torch.randn(M, N, generator=torch.Generator().manual_seed(K)).to(dtype)
    print(f"ternary bwd M={M} N={N} K={K} {dtype}", flush=True)
    gx = ops.e8t_linear_bwd_dx(gy.to(DEV), torch.from_numpy(pk).to(DEV),
                               torch.from_numpy(s16.view(np.float16).copy()).to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_bwd_f64(gy.float().numpy(), pk, s16, N, K, 32, DT_CODE[dtype])
    assert gx.shape == (M, K) and _rel(gx, ref) <= REL_TOL


@pytest.mark.parametrize("gs", [8, 16, 32, 64])
@pytest.mark.parametrize("M,N,K", SHAPES[:4] + [SHAPES[5]])
def test_2bit_bwd_mfma(gs, M, N, K):
    dtype = torch.bfloat16 if gs in (8, 32) else torch.float16
    pk, s16, _ = O.e8b_encode(_w(N, K, M + gs), gs)
    gy = torch.randn(M, N, generator=torch.Generator().manual_seed(K + gs)).to(dtype)
    print(f"2-bit bwd M={M} N={N} K={K} gs={gs}", flush=True)
    gx = ops.e8_linear_bwd_dx(gy.to(DEV), torch.from_numpy(pk).to(DEV),
                              torch.from_numpy(s16.view(np.float16).copy()).to(DEV), N, K, gs)
    torch.cuda.synchronize()
    ref = O.e8b_gemm_bwd_f64(gy.float().numpy(), pk, s16, N, K, gs, DT_CODE[dtype])
    assert gx.shape == (M, K) and _rel(gx, ref) <= REL_TOL


@pytest.mark.parametrize("gs", [8, 16, 32, 64])
@pytest.mark.parametrize("M,N,K", SHAPES[:4] + [SHAPES[5]])
def test_1bit_bwd_mfma(gs, M, N, K):
    dtype = torch.bfloat16 if gs in (16, 64) else torch.float16
    codes, s16, _ = O.e8r_encode(_w(N, K, M + 3 * gs), gs)
    gy = torch.randn(M, N, generator=torch.Generator().manual_seed(K + 7 * gs)).to(dtype)
    print(f"1-bit bwd M={M} N={N} K={K} gs={gs}", flush=True)
    gx = ops.e8r_linear_bwd_dx(gy.to(DEV), torch.from_numpy(codes).to(DEV),
                               torch.from_numpy(s16.view(np.float16).copy()).to(DEV), N, K, gs)
    torch.cuda.synchronize()
    ref = O.e8r_gemm_bwd_f64(gy.float().numpy(), codes, s16, N, K, gs, DT_CODE[dtype])
    assert gx.shape == (M, K) and _rel(gx, ref) <= REL_TOL


@pytest.mark.parametrize("fmt", ["ternary", "2bit", "1bit"])
@pytest.mark.parametrize("M,name,N,K", [(2048, "gate_up", 14336, 4096), (512, "down", 4096, 14336)])
def test_bwd_llama8b_shapes_every_element(fmt, M, name, N, K):
    gw = torch.Generator(device=DEV).manual_seed(5100 + N)
    w = torch.randn(N, K, generator=gw, device=DEV) * 0.02
    if fmt == "ternary":
        pk, sc = ops.encode(w, 32)
        wdq = ops.decode(pk, sc, N * K, 32, torch.bfloat16)
        bwd = lambda gy: ops.e8t_linear_bwd_dx(gy, pk, sc, N, K, 32)
    elif fmt == "2bit":
        pk, sc = ops.encode2(w, 32)
        wdq = ops.decode2(pk, sc, N * K, 32, torch.bfloat16)
        bwd = lambda gy: ops.e8_linear_bwd_dx(gy, pk, sc, N, K, 32)
    else:
        pk, sc = ops.encode1(w, 32)
        wdq = ops.decode1(pk, sc, N * K, 32, torch.bfloat16)
        bwd = lambda gy: ops.e8r_linear_bwd_dx(gy, pk, sc, N, K, 32)
    del w
    gy = torch.randn(M, N, generator=gw, device=DEV).to(torch.bfloat16)
    print(f"bwd {fmt} {name} M={M}", flush=True)
    gx = bwd(gy)
    ref = gy.float() @ wdq.view(N, K).float()
    torch.cuda.synchronize()
    assert torch.isfinite(gx).all()
    assert ((gx.float() - ref).abs().max() / ref.abs().max()).item() <= REL_TOL


@pytest.mark.parametrize("fmt", ["2bit", "1bit"])
@pytest.mark.parametrize("gs", [8, 16, 32, 64])
@pytest.mark.parametrize("M,N,K", [(2000, 320, 6208), (512, 1024, 4096)])
def test_lowbit_bwd_every_group_size_both_tiles(fmt, gs, M, N, K):
    # (2000, 320, 6208): 8 x 25 large tiles, unsplit, ragged rows and a last column tile
    # with 64 of its 256 output columns; (512, 1024, 4096): small tiles split over N.  Every
    # element against an fp32 matmul of the bit-exact decoded weights.
    gw = torch.Generator(device=DEV).manual_seed(5200 + gs + M)
    w = torch.randn(N, K, generator=gw, device=DEV) * 0.02
    dtype = torch.bfloat16 if gs in (8, 32) else torch.float16
    if fmt == "2bit":
        pk, sc = ops.encode2(w, gs)
        wdq = ops.decode2(pk, sc, N * K, gs, dtype)
        bwd = lambda gy: ops.e8_linear_bwd_dx(gy, pk, sc, N, K, gs)
    else:
        pk, sc = ops.encode1(w, gs)
        wdq = ops.decode1(pk, sc, N * K, gs, dtype)
        bwd = lambda gy: ops.e8r_linear_bwd_dx(gy, pk, sc, N, K, gs)
    del w
    gy = torch.randn(M, N, generator=gw, device=DEV).to(dtype)
    print(f"bwd {fmt} gs={gs} M={M} N={N} K={K}", flush=True)
    gx = bwd(gy)
    ref = gy.float() @ wdq.view(N, K).float()
    torch.cuda.synchronize()
    assert gx.shape == (M, K) and torch.isfinite(gx).all()
    assert ((gx.float() - ref).abs().max() / ref.abs().max()).item() <= REL_TOL


def test_bwd_graph_capture_matches_eager():
    # the captured launch keeps its K split (caller-owned workspace from the graph's pool):
    # every replay, with eager split work in between, is bit-identical to the eager result
    M, N, K = 64, 2048, 1024
    gw = torch.Generator(device=DEV).manual_seed(9)
    pk, sc = ops.encode(torch.randn(N, K, generator=gw, device=DEV) * 0.02, 32)
    gy = torch.randn(M, N, generator=gw, device=DEV).to(torch.bfloat16)
    eager = ops.e8t_linear_bwd_dx(gy, pk, sc, N, K, 32)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.e8t_linear_bwd_dx(gy, pk, sc, N, K, 32)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.e8t_linear_bwd_dx(gy, pk, sc, N, K, 32)
    for rep in range(3):
        out.fill_(float("nan"))
        ops.e8t_linear_bwd_dx(gy, pk, sc, N, K, 32)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
