"""Grouped decode GEMV of 1-bit Root-E8 linears (RootE8LatticePacker, ojasx2/math/lattice.py:
426-533): one launch over a whole Llama-3-8B decoder layer (seven linears, down 4096 x 14336
included) from a device job table at M = 1, 4, 5 and 16; ragged jobs at other group sizes;
the fused projections of 1-bit E8LatticeLinear layers with adapters.

Bar (north star): max|y - y_ref| / max|y_ref| <= 1e-2 against the fp64 dequantize-then-
matmul oracle with the reference's 1-bit weight rule (table[code] * scales.to(dtype),
lattice.py:511-533) on row samples, and every element against the per-linear fused op."""

import numpy as np
import pytest
import torch

import ojasx_amd
from ojasx_amd import ops
from ojasx_amd.grouped import GroupedGemv, _job
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
REL_TOL = 1e-2
LAYER = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
         ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]


def _rel(y, ref):
    y = y.detach().float().cpu().numpy() if isinstance(y, torch.Tensor) else y
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _rows_ref(x, pk, sc, K, r0, r1, gs):
    pk_np = pk.cpu().numpy()[r0 * K // 8: r1 * K // 8]
    sc_np = sc.cpu().view(torch.int16).numpy().view(np.uint16)[r0 * K // gs: r1 * K // gs]
    return O.e8r_gemm_f64(x, pk_np, sc_np, None, r1 - r0, K, gs, O.DT_BF16)


@pytest.fixture(scope="module")
def layer_gs32():
    out = []
    for j, (name, N, K) in enumerate(LAYER):
        g = torch.Generator(device=DEV).manual_seed(9750 + j)
        w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).half()
        pk, sc = ops.encode1(w, 32)
        out.append((name, N, K, pk, sc))
    return out


@pytest.mark.parametrize("M", [1, 4, 5, 16])
def test_grouped_e8r_full_decoder_layer(layer_gs32, M):
    xs = {K: torch.randn(M, K, generator=torch.Generator(device=DEV).manual_seed(9850 + M + K),
                         device=DEV).to(torch.bfloat16) for K in (4096, 14336)}
    ys = [torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
          for _, N, K, _, _ in layer_gs32]
    jobs = [_job(pk, sc, None, N, K, x=xs[K], y=y) for (_, N, K, pk, sc), y in zip(layer_gs32, ys)]
    g = GroupedGemv(jobs, M, torch.bfloat16, DEV, keep=list(xs.values()) + ys, bitrate=1.0,
                    group_size=32)
    print(f"grouped 1-bit layer M={M} grid={g.grid}", flush=True)
    for rep in range(2):
        g()
        torch.cuda.synchronize()
        for (name, N, K, pk, sc), y in zip(layer_gs32, ys):
            assert torch.isfinite(y).all(), name
            x_np = xs[K].float().cpu().numpy()
            for r0, r1 in [(0, 64), (N - 64, N)]:
                assert _rel(y[:, r0:r1], _rows_ref(x_np, pk, sc, K, r0, r1, 32)) <= REL_TOL, \
                    (name, M, r0)
            sep = ops.e8r_linear(xs[K], pk, sc, None, N, K, 32)
            assert _rel(y, sep.double().cpu().numpy()) <= REL_TOL, name


@pytest.mark.parametrize("shapes", [
    [(200, 1024), (77, 768), (1030, 2048)],   # a K % 1024 != 0: B-operand rounds at every M
    [(200, 1024), (77, 3072), (1030, 2048)],  # every K % 1024 == 0: post-scaled at M <= 4
], ids=["k256", "k1024"])
@pytest.mark.parametrize("gs", [8, 16, 64])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_grouped_e8r_group_sizes_and_ragged_jobs(gs, M, shapes):
    # ragged N, jobs sharing one output (y_col)
    layers = []
    for i, (N, K) in enumerate(shapes):
        g = torch.Generator().manual_seed(700 + i + gs)
        w = torch.randn(N, K, generator=g) * 0.02
        pk_np, sc_np = O.e8r_encode(w.numpy(), gs)[:2]
        layers.append((N, K, torch.from_numpy(pk_np).to(DEV),
                       torch.from_numpy(sc_np.view(np.float16).copy()).to(DEV), pk_np, sc_np))
    xs = {K: torch.randn(M, K, generator=torch.Generator().manual_seed(K + M)).to(torch.bfloat16)
          .to(DEV) for _, K in shapes}
    ntot = sum(N for N, _ in shapes)
    y = torch.full((M, ntot), float("nan"), dtype=torch.bfloat16, device=DEV)
    jobs, col = [], 0
    for (N, K, pk, sc, _, _) in layers:
        jobs.append(_job(pk, sc, None, N, K, x=xs[K], y=y, y_col=col, y_ld=ntot))
        col += N
    g = GroupedGemv(jobs, M, torch.bfloat16, DEV, keep=list(xs.values()) + [y], bitrate=1.0,
                    group_size=gs)
    g()
    torch.cuda.synchronize()
    col = 0
    for (N, K, _, _, pk_np, sc_np) in layers:
        ref = O.e8r_gemm_f64(xs[K].float().cpu().numpy(), pk_np, sc_np, None, N, K, gs, O.DT_BF16)
        assert _rel(y[:, col:col + N], ref) <= REL_TOL, (N, K)
        col += N


@pytest.mark.parametrize("M", [1, 16])
def test_grouped_e8r_fused_layers_with_adapters(M):
    torch.manual_seed(50 + M)
    layers = []
    for i, (n_out, rank) in enumerate([(512, 8), (128, 0), (128, 16)]):
        dense = torch.nn.Linear(1024, n_out, bias=(i != 1), device=DEV, dtype=torch.bfloat16)
        l = ojasx_amd.E8LatticeLinear.from_linear(dense, rank=rank, group_size=32, bitrate=1.0)
        if rank:
            with torch.no_grad():
                l.lora_B.normal_(0, 0.05)
        layers.append(l)
    g = GroupedGemv.fused(layers, M, torch.bfloat16)
    x = torch.randn(M, 1024, device=DEV).to(torch.bfloat16)
    y = g(x)
    torch.cuda.synchronize()
    with torch.no_grad():
        ref = torch.cat([l(x) for l in layers], dim=-1)
    assert _rel(y, ref.double().cpu().numpy()) <= REL_TOL
