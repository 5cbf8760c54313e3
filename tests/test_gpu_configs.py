"""GPU parity of the launches the benchmark times, at the benchmark's own sizes.

* one grouped decode-GEMV launch over a whole Llama-3-8B decoder layer (seven
  linears, 2,688 row tiles, so the streaming kernels run, down 4096 x 14336 included) from a
  device job table, at M = 1, 4 and 16;
* the prefill GEMM at M = 8192 on the four shapes, every element against an fp32
  matmul of the bit-exact decoded weights plus a row sample against the fp64 oracle;
* the end-to-end decoder's E8 linears at batch 4 -- fused q/k/v and gate/up
  (GroupedGemv.fused), o, down and the 128256 x 4096 lm_head -- each against the oracle;
* grouped launches of 512-1023 row tiles at 4 < M <= 16 (the K-split-by-two GEMV);
* the K-split workspace under graph capture on a side stream: a larger eager split call on
  the capture stream after capture must not disturb the graph's replays.

Bar (north star): max|y - y_ref| / max|y_ref| <= 1e-2 against the fp64 dequantize-then-matmul
oracle with the reference's weight rule (coord * scales.to(dtype), lattice.py:414-418; the
reference's own tolerance contract is tests/test_fused_e8_gemm.py:129-150).  Large layers are
checked on row samples: with K % 32 == 0 a row range is a contiguous byte range of the codes
(streaming_e8.py:182-192), so the oracle runs on that slice alone.
"""

import numpy as np
import pytest
import torch

from ojasx_amd import ops
from ojasx_amd.grouped import GroupedGemv, _job
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
REL_TOL = 1e-2
LAYER = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
         ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]


def _gpu_layer(N, K, seed):
    """W ~ N(0, 0.02) encoded on the GPU (bit-exact with the oracle: test_gpu_codec.py)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(N, K, generator=g, device=DEV) * 0.02
    pk, sc = ops.encode(w, 32)
    del w
    return pk, sc


def _np(pk, sc):
    return pk.cpu().numpy(), sc.cpu().view(torch.int16).numpy().view(np.uint16)


def _rows_ref(x, pk_np, sc_np, K, r0, r1, bias=None, dt=O.DT_BF16):
    """Oracle outputs of rows [r0, r1) of a layer (columns r0..r1 of y)."""
    n = r1 - r0
    pk = pk_np[r0 * K * 3 // 16: r1 * K * 3 // 16]
    sc = sc_np[r0 * K // 32: r1 * K // 32]
    b = None if bias is None else bias[r0:r1]
    return O.gemm_f64(x, pk, sc, b, n, K, 32, dt)


def _rel(y, ref):
    y = y.detach().float().cpu().numpy() if isinstance(y, torch.Tensor) else y
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _row_samples(N):
    return [(0, min(64, N)), (N // 2 - 32, N // 2 + 32), (N - 64, N)]


@pytest.fixture(scope="module")
def layer0():
    return [(name, N, K) + _gpu_layer(N, K, 8200 + j) for j, (name, N, K) in enumerate(LAYER)]


@pytest.mark.parametrize("copies", [1, 2])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_grouped_full_decoder_layer(layer0, M, copies):
    """the headline grouped launch (device job table, explicit x and y per job)
    over one whole decoder layer (2,688 row tiles: the staged-tile kernel at M = 1, the
    streaming kernels at M = 4 and 16) and over the layer twice (5,376 row tiles: the
    streaming kernels at every M, as in the benchmark's 224-linear stack)."""
    xs = {K: torch.randn(M, K, generator=torch.Generator(device=DEV).manual_seed(8300 + M + K),
                         device=DEV).to(torch.bfloat16) for K in (4096, 14336)}
    lin = layer0 * copies
    ys = [torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
          for _, N, K, _, _ in lin]
    jobs = [_job(pk, sc, None, N, K, x=xs[K], y=y) for (_, N, K, pk, sc), y in zip(lin, ys)]
    g = GroupedGemv(jobs, M, torch.bfloat16, DEV, keep=list(xs.values()) + ys)
    print(f"grouped layer x{copies} M={M} jobs={g.n} grid={g.grid}", flush=True)
    assert g.n == 7 * copies and sum((N + 15) // 16 for _, N, _, _, _ in lin) == 2688 * copies
    for rep in range(2):
        g()
        torch.cuda.synchronize()
        for (name, N, K, pk, sc), y in zip(lin, ys):
            assert torch.isfinite(y).all(), name
            pk_np, sc_np = _np(pk, sc)
            x_np = xs[K].float().cpu().numpy()
            for r0, r1 in _row_samples(N):
                ref = _rows_ref(x_np, pk_np, sc_np, K, r0, r1)
                assert _rel(y[:, r0:r1], ref) <= REL_TOL, (name, M, r0)
            # every element against the separate per-linear launch
            sep = ops.e8t_linear(xs[K], pk, sc, None, N, K, 32)
            assert _rel(y, sep.double().cpu().numpy()) <= REL_TOL, name


@pytest.mark.parametrize("name,N,K", [("q_o", 4096, 4096), ("k_v", 1024, 4096),
                                      ("gate_up", 14336, 4096), ("down", 4096, 14336)])
def test_prefill_m8192_full(name, N, K):
    """configs[2] at M = 8192: every element against an fp32 matmul of the decoded weights,
    and rows against the fp64 oracle."""
    M = 8192
    sid = ["q_o", "k_v", "gate_up", "down"].index(name)
    pk, sc = _gpu_layer(N, K, 8200 + sid)
    gx = torch.Generator(device=DEV).manual_seed(8400 + M)
    x = torch.randn(M, K, generator=gx, device=DEV).to(torch.bfloat16)
    print(f"prefill {name} M={M}", flush=True)
    y = ops.e8t_linear(x, pk, sc, None, N, K, 32)
    wdq = ops.decode(pk, sc, N * K, 32, torch.bfloat16).view(N, K).float()
    ref = x.float() @ wdq.t().contiguous()
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert _rel(y, ref.double().cpu().numpy()) <= REL_TOL
    del ref, wdq
    rows = [0, 1, 255, 256, 4095, 4096, M - 1]
    pk_np, sc_np = _np(pk, sc)
    ref64 = O.gemm_f64(x[rows].float().cpu().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
    assert _rel(y[rows], ref64) <= REL_TOL


class _Lin:
    """The buffers GroupedGemv.fused and E8LatticeLinear-style callers read."""

    def __init__(self, N, K, seed):
        self.packed_weight, self.block_scales = _gpu_layer(N, K, seed)
        self.out_features, self.in_features, self.group_size, self.bias = N, K, 32, None


def test_e2e_decoder_linears_batch4():
    """configs[4]'s E8 linears at batch 4, as the decoder launches them: fused q/k/v and
    gate/up (one grouped launch each), o, down and the 128256 x 4096 lm_head."""
    B, H, F, V, KV = 4, 4096, 14336, 128256, 1024
    q, k, v = _Lin(H, H, 9510), _Lin(KV, H, 9511), _Lin(KV, H, 9512)
    o, gate, up, down = _Lin(H, H, 9513), _Lin(F, H, 9514), _Lin(F, H, 9515), _Lin(H, F, 9516)
    head = _Lin(V, H, 9517)
    gx = torch.Generator(device=DEV).manual_seed(9518)
    x = (torch.randn(B, H, generator=gx, device=DEV) * 0.5).to(torch.bfloat16)
    a = (torch.randn(B, F, generator=gx, device=DEV) * 0.5).to(torch.bfloat16)
    x_np, a_np = x.float().cpu().numpy(), a.float().cpu().numpy()
    print("e2e fused qkv / gate-up", flush=True)
    for group in ([q, k, v], [gate, up]):
        gg = GroupedGemv.fused(group, B, torch.bfloat16)
        y = gg(x)
        torch.cuda.synchronize()
        col = 0
        for l in group:
            pk_np, sc_np = _np(l.packed_weight, l.block_scales)
            for r0, r1 in _row_samples(l.out_features):
                ref = _rows_ref(x_np, pk_np, sc_np, H, r0, r1)
                assert _rel(y[:, col + r0: col + r1], ref) <= REL_TOL
            col += l.out_features
    print("e2e o / down / lm_head", flush=True)
    for l, inp, inp_np in ((o, x, x_np), (down, a, a_np), (head, x, x_np)):
        y = ops.e8t_linear(inp, l.packed_weight, l.block_scales, None, l.out_features,
                           l.in_features, 32)
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
        pk_np, sc_np = _np(l.packed_weight, l.block_scales)
        for r0, r1 in _row_samples(l.out_features):
            ref = _rows_ref(inp_np, pk_np, sc_np, l.in_features, r0, r1)
            assert _rel(y[:, r0:r1], ref) <= REL_TOL, l.out_features


@pytest.mark.parametrize("M", [5, 16])
def test_grouped_512_to_1023_tiles(M):
    """A grouped launch of 600 row tiles at 4 < M <= 16 runs the in-workgroup K-split-by-two
    GEMV; every job against the oracle."""
    shapes = [(4096, 1024), (2048, 512), (3456, 256)]  # 256 + 128 + 216 = 600 tiles
    layers, xs, ys = [], {}, []
    for i, (N, K) in enumerate(shapes):
        g = torch.Generator().manual_seed(400 + i)
        w = torch.randn(N, K, generator=g) * 0.02
        pk_np, sc_np, _ = O.encode(w.numpy(), 32)
        layers.append((N, K, torch.from_numpy(pk_np).to(DEV),
                       torch.from_numpy(sc_np.view(np.float16).copy()).to(DEV), pk_np, sc_np))
        xs.setdefault(K, torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV))
        ys.append(torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV))
    jobs = [_job(pk, sc, None, N, K, x=xs[K], y=y) for (N, K, pk, sc, _, _), y in zip(layers, ys)]
    g = GroupedGemv(jobs, M, torch.bfloat16, DEV, keep=list(xs.values()) + ys)
    print(f"grouped 600 tiles M={M} grid={g.grid}", flush=True)
    g()
    torch.cuda.synchronize()
    for (N, K, _, _, pk_np, sc_np), y in zip(layers, ys):
        ref = O.gemm_f64(xs[K].float().cpu().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
        assert _rel(y, ref) <= REL_TOL, (N, K)


def test_split_workspace_survives_side_stream_capture():
    """The prefill K split's scratch comes from the caller (torch's caching allocator); a
    launch captured with torch.cuda.graph(g, stream=s) after eager warm-up on s keeps its
    own workspace in the graph's pool.  A larger eager split call on s afterwards must not
    disturb the replays, which stay bit-identical to the eager result and match the oracle."""
    K = 4096
    pk, sc = _gpu_layer(1024, K, 8201)     # k/v shape: M = 512 splits over K
    pk2, sc2 = _gpu_layer(4096, K, 8200)   # q/o shape at M = 1024: a larger split
    assert ops.workspace(ops.FMT_TERNARY, False, 512, 1024, K, 32, torch.bfloat16, DEV) is not None
    big = ops.workspace(ops.FMT_TERNARY, False, 1024, 4096, K, 32, torch.bfloat16, DEV)
    small = ops.workspace(ops.FMT_TERNARY, False, 512, 1024, K, 32, torch.bfloat16, DEV)
    assert big.numel() > small.numel()
    gx = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(512, K, generator=gx, device=DEV).to(torch.bfloat16)
    x2 = torch.randn(1024, K, generator=gx, device=DEV).to(torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = ops.e8t_linear(x, pk, sc, None, 1024, K, 32)  # warm-up on s
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        y = ops.e8t_linear(x, pk, sc, None, 1024, K, 32)
    torch.cuda.synchronize()
    pk_np, sc_np = _np(pk, sc)
    rows = [0, 1, 100, 511]
    ref = O.gemm_f64(x[rows].float().cpu().numpy(), pk_np, sc_np, None, 1024, K, 32, O.DT_BF16)
    for rep in range(3):
        with torch.cuda.stream(s):
            y2 = ops.e8t_linear(x2, pk2, sc2, None, 4096, K, 32)  # larger eager split on s
            g.replay()
        s.synchronize()
        assert torch.equal(y, eager), rep
        assert _rel(y[rows], ref) <= REL_TOL
    ref2 = O.gemm_f64(x2[:4].float().cpu().numpy(), *_np(pk2, sc2), None, 4096, K, 32,
                      O.DT_BF16)
    assert _rel(y2[:4], ref2) <= REL_TOL


@pytest.mark.parametrize("fmt", ["e8", "e8r"])
def test_strided_buffer_views(fmt):
    """Non-contiguous views of the packed codes and scales: the ops copy them, and each copy
    stays alive until the launch has been enqueued (results equal the contiguous call)."""
    N, K, M, gs = 256, 1024, 3, 32
    g = torch.Generator(device=DEV).manual_seed(7)
    w = torch.randn(N, K, generator=g, device=DEV) * 0.02
    enc, lin, bwd, dec = ((ops.encode2, ops.e8_linear, ops.e8_linear_bwd_dx, ops.decode2)
                          if fmt == "e8" else
                          (ops.encode1, ops.e8r_linear, ops.e8r_linear_bwd_dx, ops.decode1))
    pk, sc = enc(w, gs)
    # interleave with junk so the views have stride 2
    pk2 = torch.stack([pk, torch.randint_like(pk, 0, 255)], dim=1).reshape(-1)[::2]
    sc2 = torch.stack([sc, torch.rand_like(sc)], dim=1).reshape(-1)[::2]
    assert not pk2.is_contiguous() and not sc2.is_contiguous()
    x = torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16)
    gy = torch.randn(M, N, generator=g, device=DEV).to(torch.bfloat16)
    for _ in range(3):
        assert torch.equal(lin(x, pk2, sc2, None, N, K, gs), lin(x, pk, sc, None, N, K, gs))
        assert torch.equal(bwd(gy, pk2, sc2, N, K, gs), bwd(gy, pk, sc, N, K, gs))
        assert torch.equal(dec(pk2, sc2, N * K, gs, torch.bfloat16),
                           dec(pk, sc, N * K, gs, torch.bfloat16))
    # the ternary op as well
    pkt, sct = ops.encode(w, 32)
    pkt2 = torch.stack([pkt, torch.randint_like(pkt, 0, 255)], dim=1).reshape(-1)[::2]
    sct2 = torch.stack([sct, torch.rand_like(sct)], dim=1).reshape(-1)[::2]
    assert torch.equal(ops.e8t_linear(x, pkt2, sct2, None, N, K, 32),
                       ops.e8t_linear(x, pkt, sct, None, N, K, 32))
    assert torch.equal(ops.e8t_linear_bwd_dx(gy, pkt2, sct2, N, K, 32),
                       ops.e8t_linear_bwd_dx(gy, pkt, sct, N, K, 32))
