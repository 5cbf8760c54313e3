"""GPU parity of the MFMA decode GEMV (M <= 16) and of grouped launches.

Bar (north star): max|y - y_ref| / max|y_ref| <= 1e-2 against the fp64
dequantize-then-matmul oracle with the reference's bf16/fp16 weight rule
(coord * scales.to(dtype), lattice.py:414-418).  Every kernel variant (tiles per
wave R, in-workgroup K split S) is reached through the size of the launch."""

import numpy as np
import pytest
import torch

import ojasx_amd
from ojasx_amd import _native as NAT
from ojasx_amd import ops
from ojasx_amd.grouped import GroupedGemv, _job
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


def _x(M, K, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(M, K, generator=g).to(dtype)


def _rel(y, ref):
    y = y.detach().float().cpu().numpy()
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("N,K", [(256, 512), (100, 768), (16, 256), (1024, 4096)])
def test_gemv_matches_oracle(dtype, M, N, K):
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=N * 7 + K)
    x = _x(M, K, seed=M + K, dtype=dtype)
    bias = _x(1, N, seed=N, dtype=dtype).reshape(N)
    print(f"gemv M={M} N={N} K={K} {dtype}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32, DT_CODE[dtype])
    assert y.shape == (M, N) and y.dtype == dtype
    assert _rel(y, ref) <= REL_TOL


@pytest.mark.parametrize("N", [16 * 256, 16 * 512, 16 * 1024, 16 * 2048, 16 * 8192 + 48])
def test_gemv_every_variant(N):
    # per-linear launches at M = 16: < 1024 row tiles run the B-operand GEMV (gemv2m),
    # >= 1024 the streaming mask kernel; the last size also has a ragged final tile.  (The
    # in-workgroup K-split GEMV, S = 4 / 2, is reached by grouped launches of < 512 / < 1024
    # tiles: test_gpu_configs.py::test_grouped_512_to_1023_tiles and the grouped tests here.)
    K, M = 256, 16
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=N)
    x = _x(M, K, seed=3, dtype=torch.bfloat16)
    print(f"gemv variant N={N}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, None, N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
    assert _rel(y, ref) <= REL_TOL


@pytest.mark.parametrize("M", [5, 16])
@pytest.mark.parametrize("K", [768, 1280, 1536, 2048, 2560, 3328, 4608])
def test_streaming_m16_round_counts(K, M):
    # >= 1024 row tiles at 4 < M <= 16: the streaming mask kernel's 512-k rounds -- a partial
    # last round (768, 1280, 3328: lane groups past K), odd and even round counts (1536,
    # 2048), a partial last workgroup of 16 tiles (1026 tiles), and scale blocks of four
    # rounds that the rounds fill exactly (2048), cross (2560: 5 rounds, 3328: 7, 4608: 9)
    # or leave past the row's end (768 .. 1536)
    N = 16 * 1026
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=K + 7 * M)
    x = _x(M, K, seed=M + K, dtype=torch.bfloat16)
    bias = _x(1, N, seed=4, dtype=torch.bfloat16).reshape(N)
    print(f"streaming M={M} K={K}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32,
                     O.DT_BF16)
    assert _rel(y, ref) <= REL_TOL
    for m in range(M):  # each activation row against its own scale
        assert _rel(y[m:m + 1], ref[m:m + 1]) <= REL_TOL, m


def test_gemv_llama_down_shape_all_m():
    N, K = 4096, 14336
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=8206)
    for M in (1, 4, 16):
        x = _x(M, K, seed=8300 + M, dtype=torch.bfloat16)
        print(f"gemv down M={M}", flush=True)
        y = ops.e8t_linear(x.to(DEV), pk, sc, None, N, K, 32)
        torch.cuda.synchronize()
        ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
        assert _rel(y, ref) <= REL_TOL


def test_gemv_misaligned_input_uses_general_kernel():
    N, K, M = 64, 512, 3
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=5)
    xb = _x(M * K + 1, 1, seed=6, dtype=torch.bfloat16).reshape(-1).to(DEV)
    x = xb[1:].view(M, K)  # 2-byte offset: not 16-byte aligned
    y = ops.e8t_linear(x, pk, sc, None, N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().cpu().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
    assert _rel(y, ref) <= REL_TOL


class _L:  # minimal layer record for GroupedGemv.fused
    def __init__(self, N, K, seed, bias=None):
        self.packed_weight, self.block_scales, self.pk_np, self.sc_np = _encoded(N, K, seed)
        self.out_features, self.in_features, self.group_size = N, K, 32
        self.bias = bias


@pytest.mark.parametrize("M", [1, 4, 16])
def test_grouped_fused_qkv_matches_separate_linears(M):
    K = 1024
    b = _x(1, 128, seed=9, dtype=torch.bfloat16).reshape(128).to(DEV)
    layers = [_L(512, K, 11), _L(128, K, 12, bias=b), _L(128, K, 13), _L(256, K, 14)]
    x = _x(M, K, seed=M, dtype=torch.bfloat16).to(DEV)
    g = GroupedGemv.fused(layers, M, torch.bfloat16)
    print(f"grouped fused M={M} grid={g.grid}", flush=True)
    y = g(x)
    torch.cuda.synchronize()
    assert y.shape == (M, 1024)
    col = 0
    for l in layers:
        ref = O.gemm_f64(x.float().cpu().numpy(), l.pk_np, l.sc_np,
                         None if l.bias is None else l.bias.float().cpu().numpy(),
                         l.out_features, K, 32, O.DT_BF16)
        assert _rel(y[:, col:col + l.out_features], ref) <= REL_TOL
        sep = ops.e8t_linear(x, l.packed_weight, l.block_scales, l.bias, l.out_features, K, 32)
        assert _rel(y[:, col:col + l.out_features], sep.float().cpu().numpy().astype(np.float64)) <= REL_TOL
        col += l.out_features


def test_grouped_device_table_with_explicit_x_and_y():
    M = 4
    shapes = [(256, 512), (64, 1024), (300, 512), (128, 256), (512, 512), (32, 2048)]
    layers = [_L(n, k, 100 + i) for i, (n, k) in enumerate(shapes)]
    xs = {k: _x(M, k, seed=k, dtype=torch.float16).to(DEV) for k in {k for _, k in shapes}}
    ys = [torch.full((M, n), float("nan"), dtype=torch.float16, device=DEV) for n, _ in shapes]
    jobs = [_job(l.packed_weight, l.block_scales, None, l.out_features, l.in_features,
                 x=xs[l.in_features], y=y) for l, y in zip(layers, ys)]
    g = GroupedGemv(jobs, M, torch.float16, DEV, keep=list(xs.values()) + ys)
    print(f"grouped table jobs={g.n} grid={g.grid}", flush=True)
    for _ in range(2):  # replaying a planned table is idempotent
        g()
        torch.cuda.synchronize()
        for l, y in zip(layers, ys):
            ref = O.gemm_f64(xs[l.in_features].float().cpu().numpy(), l.pk_np, l.sc_np, None,
                             l.out_features, l.in_features, 32, O.DT_F16)
            assert _rel(y, ref) <= REL_TOL


def test_grouped_plan_rejects_bad_jobs():
    l = _L(64, 512, 1)
    bad_k = _job(l.packed_weight, l.block_scales, None, 64, 500)
    with pytest.raises(RuntimeError, match="K % 256"):
        GroupedGemv([bad_k], 4, torch.bfloat16, DEV)
    ok = _job(l.packed_weight, l.block_scales, None, 64, 512)
    with pytest.raises(RuntimeError, match="1 <= M <= 16"):
        GroupedGemv([ok], 17, torch.bfloat16, DEV)
    g = GroupedGemv([ok], 2, torch.bfloat16, DEV, keep=[l.packed_weight, l.block_scales])
    with pytest.raises(RuntimeError, match="no activations"):
        g()


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 16])
@pytest.mark.parametrize("K", [1280, 4096])
def test_wide_kernel_partial_rounds_and_ragged_rows(M, K):
    # >= 1024 row tiles selects the streaming kernel; K = 1280 leaves a partial
    # second round (one live chunk of four), N = 16424 a ragged last tile
    N = 16 * 1024 + 40
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=K + M)
    x = _x(M, K, seed=M * 3, dtype=torch.bfloat16)
    bias = _x(1, N, seed=4, dtype=torch.bfloat16).reshape(N)
    print(f"wide M={M} K={K}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32, O.DT_BF16)
    assert _rel(y, ref) <= REL_TOL


@pytest.mark.parametrize("M", [1, 3, 4])
@pytest.mark.parametrize("K", [3072, 3328, 5120])
def test_post_scaled_scale_pairs_round_counts(M, K):
    # the post-scaled streaming kernel (two tiles per wave) fetches the scales of rounds 2v
    # and 2v + 1 together: odd round counts (3072: 3 rounds, 5120: 5) end on a pair whose
    # second round does not exist, 3328 (3.25 rounds) on a partial round in a pair's second
    # half; 4099 row tiles keep it on that kernel at M = 3 and 4.  The layer is encoded on
    # the GPU (bit-exact with the oracle's encoder, test_gpu_codec.py); every element is
    # checked against an fp32 matmul of the decoded weights and row samples against the
    # fp64 oracle.
    N = 4 * 16 * 1024 + 40
    w = torch.randn(N, K, generator=torch.Generator(device=DEV).manual_seed(3 * K + M),
                    device=DEV) * 0.02
    pk, sc = ops.encode(w, 32)
    del w
    x = _x(M, K, seed=M * 7 + K, dtype=torch.bfloat16)
    bias = _x(1, N, seed=8, dtype=torch.bfloat16).reshape(N)
    print(f"post-scaled scale pairs M={M} K={K}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    dense = ops.decode(pk, sc, N * K, 32, torch.bfloat16).view(N, K).float()
    full = x.to(DEV).float() @ dense.t() + bias.to(DEV).float()
    del dense
    assert _rel(y, full.double().cpu().numpy()) <= REL_TOL
    pk_np, sc_np = pk.cpu().numpy(), sc.cpu().view(torch.int16).numpy().view(np.uint16)
    for r0, r1 in [(0, 64), (N // 2 - 32, N // 2 + 32), (N - 64, N)]:
        ref = O.gemm_f64(x.float().numpy(), pk_np[r0 * K * 3 // 16: r1 * K * 3 // 16],
                         sc_np[r0 * K // 32: r1 * K // 32], bias[r0:r1].float().numpy(),
                         r1 - r0, K, 32, O.DT_BF16)
        assert _rel(y[:, r0:r1], ref) <= REL_TOL, r0
        for m in range(M):  # each activation row against its own reference
            assert _rel(y[m:m + 1, r0:r1], ref[m:m + 1]) <= REL_TOL, (r0, m)


@pytest.mark.parametrize("M", [2, 4])
@pytest.mark.parametrize("K", [1024, 3072, 4608, 9216])
def test_wide_one_tile_per_wave_round_counts(M, K):
    # 1024..4095 row tiles at 1 < M <= 4: the streaming kernel with one row tile per wave, at
    # one to nine rounds per wave (4608: a partial fifth round)
    N = 16 * 1024 + 40
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=2 * K + M)
    x = _x(M, K, seed=M * 5 + K, dtype=torch.bfloat16)
    bias = _x(1, N, seed=6, dtype=torch.bfloat16).reshape(N)
    print(f"wide one tile per wave M={M} K={K}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32, O.DT_BF16)
    assert _rel(y, ref) <= REL_TOL
    for m in range(M):  # each activation row against its own reference
        assert _rel(y[m:m + 1], ref[m:m + 1]) <= REL_TOL, m


@pytest.mark.parametrize("M", [1, 2, 4])
def test_wide_bf16_activation_dynamic_range(M):
    # activations with a wide dynamic range through the streaming kernels at M <= 4:
    # outliers (x1000), tiny values (x1e-3), blocks of zeros, a block of 1e-30 and a row far
    # larger than the others; each row stays within the bar against its own scale
    N, K = 16 * 1024 + 16, 2048
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=91)
    g = torch.Generator().manual_seed(92)
    x = torch.randn(M, K, generator=g)
    idx = torch.randperm(M * K, generator=g)
    x.view(-1)[idx[: M * K // 100]] *= 1000.0
    x.view(-1)[idx[M * K // 100: M * K // 50]] *= 1e-3
    x[:, 64:96] = 0.0
    x[0, 1000:1032] = 1e-30
    if M > 1:
        x[1] *= 1e6
    x = x.to(torch.bfloat16)
    print(f"dynamic range M={M}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, None, N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
    for m in range(M):  # each row against its own scale
        assert _rel(y[m:m + 1], ref[m:m + 1]) <= REL_TOL, m


@pytest.mark.parametrize("M", [4, 12])
def test_wide_kernel_fp16_and_subnormal_scales(M):
    # tiny weights give fp16-subnormal group scales; fp16 activations keep them exactly
    # (M = 4: post-scaled kernel, M = 12: mask kernel)
    N, K = 16 * 1024, 512
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=77, scale=2e-6)
    assert (np.abs(sc_np.view(np.float16).astype(np.float32)) < 6.1e-5).mean() > 0.5
    x = _x(M, K, seed=78, dtype=torch.float16)
    y = ops.e8t_linear(x.to(DEV), pk, sc, None, N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_F16)
    assert _rel(y, ref) <= REL_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K", [(1, 1024), (3, 1024), (1, 2048), (4, 3072), (2, 8192),
                                 (4, 8192), (1, 12288), (1, 16384)])
def test_staged_tile_gemv_round_counts(dtype, M, K):
    # per-linear launches of fewer than 1024 row tiles at M <= 4 and K % 1024 == 0 run the
    # staged-tile kernel: 1..16 rounds of 1024 k over 4 waves (idle waves for K < 4096,
    # up to 4 rounds per wave), ragged last tile, bias
    N = 16 * 37 + 9
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=K + M)
    x = _x(M, K, seed=M * 11 + K, dtype=dtype)
    bias = _x(1, N, seed=5, dtype=dtype).reshape(N)
    print(f"staged tile M={M} K={K} {dtype}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32,
                     DT_CODE[dtype])
    assert _rel(y, ref) <= REL_TOL


@pytest.mark.parametrize("K", [1024, 4096])
def test_staged_tile_gemv_two_tile_workgroups(K):
    # 777 row tiles at M = 1 (two tiles per workgroup): an odd tile count, so the last
    # workgroup's second tile lies past N, and a ragged last tile
    N = 16 * 776 + 7
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=N + K)
    x = _x(1, K, seed=K, dtype=torch.bfloat16)
    print(f"staged tile pairs N={N} K={K}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, None, N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_BF16)
    assert _rel(y, ref) <= REL_TOL


@pytest.mark.parametrize("M", [2, 3, 4])
def test_staged_tile_gemv_two_tiles_per_wave(M):
    # 777 row tiles at 1 < M <= 4 run two row tiles per wave: an odd tile count, so the last
    # wave's second tile lies past N, and a ragged last tile, with bias
    N, K = 16 * 776 + 7, 4096
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=N + M)
    x = _x(M, K, seed=M * 3 + 1, dtype=torch.bfloat16)
    bias = _x(1, N, seed=8, dtype=torch.bfloat16).reshape(N)
    print(f"staged tile two tiles per wave M={M}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32, O.DT_BF16)
    assert _rel(y, ref) <= REL_TOL


@pytest.mark.parametrize("M", [2, 3])
def test_gemv_down_shape_small_layer_kernel(M):
    # K = 14336 at 1 < M <= 4: the small-layer post-scaled kernel (8 waves per workgroup,
    # 14 rounds per tile: two on the first six waves, one on the last two)
    N, K = 4096, 14336
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=8206 + M)
    x = _x(M, K, seed=8400 + M, dtype=torch.float16)
    print(f"gemv down small-layer kernel M={M}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, None, N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, None, N, K, 32, O.DT_F16)
    assert _rel(y, ref) <= REL_TOL


@pytest.mark.parametrize("M", [2, 3, 4])
def test_grouped_mid_size_launch_one_tile_per_wave(M):
    # grouped launches of 1024..4095 row tiles at 1 < M <= 4 stream with one row tile per
    # wave (the decoder's fused gate/up: 2 x 896 tiles); ragged second job
    K = 4096
    layers = [_L(14336, K, 31), _L(14336 - 40, K, 32)]
    x = _x(M, K, seed=40 + M, dtype=torch.bfloat16).to(DEV)
    g = GroupedGemv.fused(layers, M, torch.bfloat16)
    print(f"grouped mid-size M={M} grid={g.grid}", flush=True)
    y = g(x)
    torch.cuda.synchronize()
    col = 0
    for l in layers:
        ref = O.gemm_f64(x.float().cpu().numpy(), l.pk_np, l.sc_np, None, l.out_features, K, 32,
                         O.DT_BF16)
        assert _rel(y[:, col:col + l.out_features], ref) <= REL_TOL
        col += l.out_features


@pytest.mark.parametrize("M", [5, 12, 16])
@pytest.mark.parametrize("N,K", [(100, 1280), (16 * 300 + 5, 2304), (16 * 600 + 9, 1280),
                                 (100, 4352), (16 * 40 + 3, 6400), (48, 16384)])
def test_per_linear_b_operand_resident_and_prefetched(M, N, K):
    # per-linear 4 < M <= 16 launches below 1024 row tiles: K <= 4096 stages the activations
    # once per workgroup (1, 2 or 4 row tiles per workgroup by the tile count; rounds past K
    # on some waves), 4096 < K <= 16384 prefetches every round's weights (waves with one
    # round more than others at K = 4352; all eight rounds per wave at K = 16384); ragged N
    pk, sc, pk_np, sc_np = _encoded(N, K, seed=N + 3 * K + M)
    x = _x(M, K, seed=5 * M + K, dtype=torch.bfloat16)
    bias = _x(1, N, seed=N + 1, dtype=torch.bfloat16).reshape(N)
    print(f"b-operand per-linear M={M} N={N} K={K}", flush=True)
    y = ops.e8t_linear(x.to(DEV), pk, sc, bias.to(DEV), N, K, 32)
    torch.cuda.synchronize()
    ref = O.gemm_f64(x.float().numpy(), pk_np, sc_np, bias.float().numpy(), N, K, 32, O.DT_BF16)
    assert _rel(y, ref) <= REL_TOL
    for m in range(M):
        assert _rel(y[m:m + 1], ref[m:m + 1]) <= REL_TOL, m
