"""The allocation-free forward (ojx_e8t_gemm_fwd_noalloc) against ojx_e8t_gemm_fwd.

Both run the same kernels with the same K split (the static scratch is at least as large as
the workspace each shape needs), so their outputs are bit-identical; both are also checked
against the fp64 oracle at the north star's bar (max|y - y_ref| / max|y_ref| <= 1e-2).  Two
calls in a row, the second smaller, share the static scratch; a shape whose split needs more
scratch than the array holds is refused before any launch."""

import ctypes

import numpy as np
import pytest
import torch

from ojasx_amd import _native as N
from ojasx_amd import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
STATIC_SCRATCH = 64 << 20


def _need(M, N_out, K):
    n = ctypes.c_size_t(0)
    N.check(N.lib().ojx_gemm_workspace_bytes(0, 0, M, N_out, K, 32, N.BF16, ctypes.byref(n)),
            "workspace query")
    return n.value


def _layer(N_out, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(N_out, K, generator=g, device=DEV) * 0.02
    return ops.encode(w, 32)


def _with_workspace(x, pk, sc, M, N_out, K):
    y = torch.full((M, N_out), float("nan"), dtype=torch.bfloat16, device=DEV)
    ws = ops.workspace(ops.FMT_TERNARY, False, M, N_out, K, 32, torch.bfloat16, DEV)
    N.check(N.lib().ojx_e8t_gemm_fwd(x.data_ptr(), pk.data_ptr(), sc.data_ptr(), None,
                                     y.data_ptr(), M, N_out, K, 32, N.BF16,
                                     None if ws is None else ws.data_ptr(),
                                     0 if ws is None else ws.numel(),
                                     torch.cuda.current_stream().cuda_stream), "gemm_fwd")
    torch.cuda.synchronize()
    return y


def _noalloc(x, pk, sc, M, N_out, K):
    y = torch.full((M, N_out), float("nan"), dtype=torch.bfloat16, device=DEV)
    N.check(N.lib().ojx_e8t_gemm_fwd_noalloc(x.data_ptr(), pk.data_ptr(), sc.data_ptr(), None,
                                             y.data_ptr(), M, N_out, K, 32, N.BF16,
                                             torch.cuda.current_stream().cuda_stream),
            "gemm_fwd_noalloc")
    torch.cuda.synchronize()
    return y


def test_noalloc_matches_workspace_entry_point_on_two_calls():
    K = 4096
    cases = [(512, 4096, 8200), (64, 1024, 8201)]  # second call smaller; both split over K
    for M, N_out, seed in cases:
        need = _need(M, N_out, K)
        assert 0 < need <= STATIC_SCRATCH
        pk, sc = _layer(N_out, K, seed)
        gx = torch.Generator(device=DEV).manual_seed(seed + 1)
        x = torch.randn(M, K, generator=gx, device=DEV).to(torch.bfloat16)
        print(f"noalloc M={M} N={N_out} K={K} scratch={need}", flush=True)
        y0 = _noalloc(x, pk, sc, M, N_out, K)
        y1 = _with_workspace(x, pk, sc, M, N_out, K)
        assert torch.isfinite(y0).all()
        assert torch.equal(y0, y1)
        rows = [0, 1, M // 2, M - 1]
        ref = O.gemm_f64(x[rows].float().cpu().numpy(), pk.cpu().numpy(),
                         sc.cpu().view(torch.int16).numpy().view(np.uint16), None, N_out, K, 32,
                         O.DT_BF16)
        got = y0[rows].float().cpu().numpy()
        assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-2


def test_noalloc_decode_shape_needs_no_scratch():
    M, N_out, K = 4, 1024, 4096
    assert _need(M, N_out, K) == 0
    pk, sc = _layer(N_out, K, 8202)
    x = torch.randn(M, K, generator=torch.Generator(device=DEV).manual_seed(3),
                    device=DEV).to(torch.bfloat16)
    assert torch.equal(_noalloc(x, pk, sc, M, N_out, K), _with_workspace(x, pk, sc, M, N_out, K))


def test_noalloc_refuses_shapes_beyond_the_static_scratch():
    M, N_out, K = 512, 20480, 4096  # a large-tile split of 2 x 512 x 20480 fp32 = 80 MiB
    assert _need(M, N_out, K) > STATIC_SCRATCH
    st = N.lib().ojx_e8t_gemm_fwd_noalloc(None, None, None, None, None, M, N_out, K, 32,
                                          N.BF16, None)
    assert st == -2
    assert b"static scratch" in N.lib().ojx_e8t_last_error()
