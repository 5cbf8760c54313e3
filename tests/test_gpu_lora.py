"""GPU parity of the fused LoRA epilogue (E8LatticeLinear with rank > 0).

The reference adds the adapter after the E8 op: out + scaling * ((x @ A) @ B)
(ojasx2/math/lattice.py:839-842).  The fused forward adds the same term inside the E8
kernel's epilogue, so it is checked against the fp64 oracle of the E8 op plus the adapter
term in fp64, at the north star's bar (max|y - y_ref| / max|y_ref| <= 1e-2 for bf16/fp16;
abs 1e-4 for fp32, the reference test's tolerance, tests/test_fused_e8_gemm.py:129-150).
Every forward route is reached: the staged-tile and B-operand GEMVs, the 2-bit GEMV, the
MFMA prefill GEMM (with and without its K split), the general kernel and grouped launches.
Gradients (x through the fused backward, A, B and bias in torch) are checked against
torch autograd in fp64 on the oracle's decoded weights."""

import numpy as np
import pytest
import torch

import ojasx_amd
from ojasx_amd import ops
from ojasx_amd.grouped import GroupedGemv
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
DT_CODE = {torch.float16: O.DT_F16, torch.bfloat16: O.DT_BF16, torch.float32: O.DT_F32}
FMTS = {  # format: (encoder, oracle gemm, oracle decode)
    ops.FMT_TERNARY: (O.encode, O.gemm_f64, O.decode),
    ops.FMT_E8: (O.e8b_encode, O.e8b_gemm_f64, O.e8b_decode),
    ops.FMT_ROOT: (O.e8r_encode, O.e8r_gemm_f64, O.e8r_decode),
}


def _layer(fmt, N, K, gs, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    pk, s16, _ = FMTS[fmt][0](w.numpy(), gs)
    return (torch.from_numpy(pk).to(DEV), torch.from_numpy(s16.view(np.float16).copy()).to(DEV),
            pk, s16)


def _ref(fmt, x, pk, s16, bias, a, b, scaling, N, K, gs, dtype):
    y = FMTS[fmt][1](x.float().cpu().numpy(), pk, s16,
                     None if bias is None else bias.float().cpu().numpy(), N, K, gs,
                     DT_CODE[dtype])
    x64 = x.double().cpu().numpy().reshape(-1, K)
    return y + scaling * (x64 @ a.double().cpu().numpy()) @ b.double().cpu().numpy()


def _check(y, ref, dtype):
    y = y.detach().double().cpu().numpy().reshape(ref.shape)
    if dtype == torch.float32:
        assert np.abs(y - ref).max() <= 1e-4
    else:
        assert np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30) <= 1e-2


@pytest.mark.parametrize("fmt", [ops.FMT_TERNARY, ops.FMT_E8, ops.FMT_ROOT])
@pytest.mark.parametrize("M", [1, 4, 7, 16, 64, 600])
def test_fused_lora_matches_oracle_plus_adapter(fmt, M):
    N, K, gs, r, scaling = 1024 + 16 * 3, 2048, 32, 8, 2.0
    pk, sc, pk_np, s16 = _layer(fmt, N, K, gs, seed=fmt * 100 + M)
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    a = (torch.randn(K, r, generator=g) * 0.05).to(torch.bfloat16)
    b = (torch.randn(r, N, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    print(f"lora fmt={fmt} M={M}", flush=True)
    y = ops.linear_lora(x.to(DEV), pk, sc, bias.to(DEV), a.to(DEV), b.to(DEV), scaling, fmt, N,
                        K, gs)
    torch.cuda.synchronize()
    _check(y, _ref(fmt, x, pk_np, s16, bias, a, b, scaling, N, K, gs, torch.bfloat16),
           torch.bfloat16)


@pytest.mark.parametrize("r", [1, 16, 24, 64])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_fused_lora_ranks_and_dtypes(r, dtype):
    # fp32 activations run the general kernel; fp16 the fast routes
    N, K, M, gs, scaling = 256, 1024, 5, 32, 0.5
    pk, sc, pk_np, s16 = _layer(ops.FMT_TERNARY, N, K, gs, seed=r)
    g = torch.Generator().manual_seed(r)
    x = torch.randn(M, K, generator=g).to(dtype)
    a = (torch.randn(K, r, generator=g) * 0.05).to(dtype)
    b = (torch.randn(r, N, generator=g) * 0.05).to(dtype)
    y = ops.linear_lora(x.to(DEV), pk, sc, None, a.to(DEV), b.to(DEV), scaling,
                        ops.FMT_TERNARY, N, K, gs)
    torch.cuda.synchronize()
    _check(y, _ref(ops.FMT_TERNARY, x, pk_np, s16, None, a, b, scaling, N, K, gs, dtype), dtype)


def test_fused_lora_prefill_split_and_graph():
    # M = 512 on a k/v-shaped layer: the MFMA GEMM split over K (the adapter term is added by
    # the split's reduction kernel); the same launch captured into a graph replays identically
    N, K, M, gs, r, scaling = 1024, 4096, 512, 32, 8, 2.0
    assert ops.workspace(ops.FMT_TERNARY, False, M, N, K, gs, torch.bfloat16, DEV) is not None
    pk, sc, pk_np, s16 = _layer(ops.FMT_TERNARY, N, K, gs, seed=77)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    a = (torch.randn(K, r, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    b = (torch.randn(r, N, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    eager = ops.linear_lora(x, pk, sc, None, a, b, scaling, ops.FMT_TERNARY, N, K, gs)
    torch.cuda.synchronize()
    rows = [0, 1, 255, 511]
    ref = _ref(ops.FMT_TERNARY, x[rows].cpu(), pk_np, s16, None, a.cpu(), b.cpu(), scaling, N, K,
               gs, torch.bfloat16)
    _check(eager[rows], ref, torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.linear_lora(x, pk, sc, None, a, b, scaling, ops.FMT_TERNARY, N, K, gs)
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        y = ops.linear_lora(x, pk, sc, None, a, b, scaling, ops.FMT_TERNARY, N, K, gs)
    for _ in range(3):
        with torch.cuda.stream(s):
            graph.replay()
        s.synchronize()
        assert torch.equal(y, eager)


@pytest.mark.parametrize("bitrate", [1.5, 2.0, 1.0])
def test_lora_layer_gradients(bitrate):
    # E8LatticeLinear with an adapter: forward through the fused op, gradients for x, A, B
    # and bias against torch autograd in fp64 on the decoded weights
    K, N, M, r = 512, 256, 6, 8
    torch.manual_seed(5)
    lin = torch.nn.Linear(K, N, bias=True)
    layer = ojasx_amd.E8LatticeLinear.from_linear(lin, rank=r, lora_alpha=16.0, group_size=32,
                                                  bitrate=bitrate).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        layer.lora_B.copy_(torch.randn(r, N) * 0.05)
    x = torch.randn(M, K, device=DEV).to(torch.bfloat16).requires_grad_(True)
    y = layer(x)
    gy = torch.randn(M, N, device=DEV).to(torch.bfloat16)
    y.backward(gy)
    torch.cuda.synchronize()
    w = layer.unpack_weights(torch.bfloat16).double().cpu()
    x64 = x.detach().double().cpu().requires_grad_(True)
    a64 = layer.lora_A.detach().double().cpu().requires_grad_(True)
    b64 = layer.lora_B.detach().double().cpu().requires_grad_(True)
    bias64 = layer.bias.detach().double().cpu().requires_grad_(True)
    y64 = x64 @ w.t() + bias64 + layer.scaling * (x64 @ a64) @ b64
    y64.backward(gy.double().cpu())

    def rel(got, ref):
        got = got.detach().double().cpu()
        return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()

    assert rel(y, y64.detach()) <= 1e-2
    assert rel(x.grad, x64.grad) <= 1e-2
    assert rel(layer.lora_A.grad, a64.grad) <= 1e-2
    assert rel(layer.lora_B.grad, b64.grad) <= 1e-2
    assert rel(layer.bias.grad, bias64.grad) <= 1e-2


def test_grouped_fused_projection_with_adapters():
    # q/k/v in one grouped launch with adapters on q and v (configs[4]'s layout): equals the
    # separate fused layers
    K, M = 1024, 4
    layers = []
    for i, n in enumerate((512, 128, 128)):
        lin = torch.nn.Linear(K, n, bias=False)
        torch.manual_seed(i)
        lyr = ojasx_amd.E8LatticeLinear.from_linear(lin, rank=8 if i != 1 else 0,
                                                    lora_alpha=16.0, group_size=32,
                                                    bitrate=1.5).to(DEV).to(torch.bfloat16)
        if lyr.rank:
            with torch.no_grad():
                lyr.lora_B.copy_(torch.randn(8, n) * 0.05)
        layers.append(lyr)
    x = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    g = GroupedGemv.fused(layers, M, torch.bfloat16)
    with torch.no_grad():
        y = g(x)
        torch.cuda.synchronize()
        col = 0
        for l in layers:
            sep = l(x)
            ref = sep.double()
            got = y[:, col:col + l.out_features].double()
            assert ((got - ref).abs().max() / ref.abs().max()).item() <= 1e-2
            col += l.out_features


@pytest.mark.parametrize("r", [8, 16])
@pytest.mark.parametrize("K", [1024, 4096])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_fused_lora_tile_route_u_in_launch(M, K, r):
    # per-linear decode on the staged-tile route: a rank-8 adapter's u is formed inside the
    # GEMV launch (each wave adds its own round's k range; at K = 1024 three of the four
    # waves have none), a rank-16 one by the separate down-projection launch first
    N, gs, scaling = 512 + 16, 32, 2.0
    pk, sc, pk_np, s16 = _layer(ops.FMT_TERNARY, N, K, gs, seed=1000 + 10 * M + K // 1024 + r)
    g = torch.Generator().manual_seed(M + K + r)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    a = (torch.randn(K, r, generator=g) * 0.05).to(torch.bfloat16)
    b = (torch.randn(r, N, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    print(f"lora tile M={M} K={K} r={r}", flush=True)
    y = ops.linear_lora(x.to(DEV), pk, sc, bias.to(DEV), a.to(DEV), b.to(DEV), scaling,
                        ops.FMT_TERNARY, N, K, gs)
    torch.cuda.synchronize()
    _check(y, _ref(ops.FMT_TERNARY, x, pk_np, s16, bias, a, b, scaling, N, K, gs,
                   torch.bfloat16), torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1, 4])
def test_grouped_adapters_u_in_launch_against_oracle(M, dtype):
    # configs[4]'s q/k/v at K = 4096 in one grouped launch (staged-tile kernel, one round per
    # wave): the rank-8 adapters of q and v are formed inside the launch; every output
    # column against the fp64 oracle of the E8 op plus the adapter term
    K, gs, scaling = 4096, 32, 2.0
    shapes = ((1024, 8), (256, 0), (256, 8))
    layers, refs_in = [], []
    for i, (n, r) in enumerate(shapes):
        pk, sc, pk_np, s16 = _layer(ops.FMT_TERNARY, n, K, gs, seed=2000 + i)
        g = torch.Generator().manual_seed(2100 + i)
        a = (torch.randn(K, max(r, 1), generator=g) * 0.05).to(dtype)
        b = (torch.randn(max(r, 1), n, generator=g) * 0.05).to(dtype)
        lyr = type("L", (), {})()
        lyr.packed_weight, lyr.block_scales, lyr.bias = pk, sc, None
        lyr.out_features, lyr.in_features, lyr.group_size, lyr.bitrate = n, K, gs, 1.5
        lyr.rank = r
        if r:
            lyr.lora_A, lyr.lora_B, lyr.scaling = a.to(DEV), b.to(DEV), scaling
        layers.append(lyr)
        refs_in.append((pk_np, s16, n, r, a, b))
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(dtype)
    grp = GroupedGemv.fused(layers, M, dtype)
    y = grp(x.to(DEV))
    torch.cuda.synchronize()
    col = 0
    for pk_np, s16, n, r, a, b in refs_in:
        if r:
            ref = _ref(ops.FMT_TERNARY, x, pk_np, s16, None, a, b, scaling, n, K, gs, dtype)
        else:
            ref = O.gemm_f64(x.float().numpy(), pk_np, s16, None, n, K, gs, DT_CODE[dtype])
        _check(y[:, col:col + n], ref, dtype)
        col += n
