"""Host logic of the ``ojasx3.hardware`` entry (ojasx_amd.hardware; tilelang_kernels.py:75-177,
426-615, tile_fallback.py:25-52): no GPU needed.

* ``select_tile_config``: the reference's ROCm rows of its own parametrised test
  (tests/test_emitted_cpu_kernel.py:117-131) plus the fp32 branch and the error types;
* the dense call and the ReLU^2 + ballot form against ``F.linear`` and a bit-by-bit
  loop over the columns (a wrong shift, word or padding fails it);
* the packed call's argument errors.
"""

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from ojasx_amd import hardware as H


@pytest.mark.parametrize("device,M,N,K,dtype,tile", [
    ("rocm", 32, 128, 128, torch.float16, (64, 64, 32, 4)),       # reference test row
    ("rocm", 256, 256, 256, torch.bfloat16, (128, 128, 32, 8)),   # reference test row
    ("cuda", 32, 128, 128, torch.float16, (64, 64, 32, 4)),
    ("cuda:0", 256, 256, 256, torch.float16, (128, 128, 32, 8)),
    ("auto", 128, 128, 64, torch.bfloat16, (128, 128, 32, 8)),
    ("hip", 128, 127, 64, torch.bfloat16, (64, 64, 32, 4)),
    ("gfx950", 128, 128, 64, torch.float32, (64, 64, 32, 4)),      # fp32 needs M, N >= 256
    ("gfx950", 256, 256, 64, torch.float32, (128, 128, 32, 8)),
    (torch.device("cuda"), 128, 128, 64, "float16", (128, 128, 32, 8)),
    ("rocm", 128, 128, 64, "fp32", (64, 64, 32, 4)),
    ("rocm", 128, 128, 64, "int8", (128, 128, 32, 8)),
    ("rocm", 128, 128, 64, None, (128, 128, 32, 8)),
])
def test_select_tile_config_rocm_rows(device, M, N, K, dtype, tile):
    cfg = H.TileLangHardwareAutoTuner.select_tile_config(M, N, K, device=device, dtype=dtype)
    assert tuple(cfg[:4]) == tile and cfg.target_arch == "rocm"
    assert cfg.to_dict()["block_k"] == 32


@pytest.mark.parametrize("dims", [(0, 1, 1), (1, -1, 1), (1, 1, 0)])
def test_select_tile_config_rejects_nonpositive(dims):
    with pytest.raises(ValueError):
        H.TileLangHardwareAutoTuner.select_tile_config(*dims, device="rocm")


@pytest.mark.parametrize("arch", ["mps", "metal", "sycl", "xpu", "ascend", "cpu", "sm90"])
def test_other_architectures_are_refused(arch):
    with pytest.raises(RuntimeError, match="Unsupported target_arch"):
        H.TileLangHardwareAutoTuner.select_tile_config(64, 64, 64, device=arch)
    with pytest.raises(RuntimeError):
        H.compile_or_emit_universal_kernel(64, 64, 64, device=arch)


def test_kernel_record_and_source():
    k = H.compile_or_emit_universal_kernel(2048, 4096, 4096, device="rocm", bitrate=1.5,
                                           group_size=32, dtype=torch.bfloat16)
    assert (k.M, k.N, k.K, k.block_m, k.block_n, k.block_k) == (2048, 4096, 4096, 128, 128, 32)
    assert k.target_arch == "rocm" and k.backend == "hip_gfx950" and k.bitrate == 1.5
    assert k["panel_size"] == 8 and k["callable"] is k
    assert "ojx_e8t_gemm_fwd" in k and "MFMA" in str(k) and "tile_config" in k
    assert "ojx_e8r_gemm_fwd" in H.compile_or_emit_universal_kernel(1, 64, 64, bitrate=1.0)
    d = H.compile_or_emit_universal_kernel(4, 64, 64, bitrate=2.0)
    assert "ojx_e8_gemm_fwd" in d and "decode GEMV" in d.source
    assert H.is_tilelang_available() is False


def _mask_by_loop(z):
    rows, cols = z.shape
    words = (cols + 31) // 32
    out = torch.zeros(rows, words, dtype=torch.int64)
    for r in range(rows):
        for c in range(cols):
            if z[r, c] > 0:
                out[r, c // 32] |= 1 << (c % 32)
    out = torch.where(out >= 2 ** 31, out - 2 ** 32, out)  # int32 two's complement
    return out.to(torch.int32)


@pytest.mark.parametrize("N", [1, 31, 32, 33, 70])
def test_dense_call_and_relu2_ballot(N):
    g = torch.Generator().manual_seed(N)
    M, K = 5, 24
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g)
    b = torch.randn(N, generator=g)
    k = H.compile_or_emit_universal_kernel(M, N, K, device="rocm", dtype=torch.float32)
    torch.testing.assert_close(k(x, w, b), F.linear(x, w, b), rtol=0, atol=0)
    torch.testing.assert_close(k(x, w, None, b), F.linear(x, w, b), rtol=0, atol=0)
    y, mask = k(x, w, b, relu2_ballot=True)
    z = F.linear(x, w, b)
    torch.testing.assert_close(y, F.relu(z).square(), rtol=0, atol=0)
    assert mask.dtype == torch.int32 and mask.shape == (M, (N + 31) // 32)
    assert torch.equal(mask, _mask_by_loop(z))
    y2, mask2 = k.forward_relu2_ballot(x, w, b)
    assert torch.equal(y2, y) and torch.equal(mask2, mask)


def test_module_call_uses_forward():
    lin = nn.Linear(16, 8)
    x = torch.randn(3, 16)
    k = H.compile_or_emit_universal_kernel(3, 8, 16)
    torch.testing.assert_close(k(x, lin), lin(x))


def test_packed_call_argument_errors():
    k = H.compile_or_emit_universal_kernel(2, 64, 64, bitrate=1.5)
    packed = torch.zeros(64 * 64 * 3 // 16, dtype=torch.uint8)
    with pytest.raises(ValueError, match="block_scales"):
        k(torch.randn(2, 64), packed)
    with pytest.raises(RuntimeError, match="HIP device"):
        k(torch.randn(2, 64), packed, torch.ones(128, dtype=torch.float16))
    assert H.dispatch_tilelang_e8_gemm(torch.randn(2, 64), packed,
                                       torch.ones(128, dtype=torch.float16), None, 64, 64, 32,
                                       1.5) is None
