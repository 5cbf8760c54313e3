"""GPU parity of the encoder and decoder kernels against the CPU oracle.

Bar: bit-exact codes, scales and decoded weights (integer/byte work).  Small and
edge cases compare element by element; the BASELINE configs compare whole
layers (C1: 4096x4096 fp32 seed 8101; C4: a 14336x4096 fp16 layer with 0.1%
+-8 sigma outliers), plus size-independent round-trip properties."""

import numpy as np
import pytest
import torch

import ojasx_amd
from ojasx_amd import ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _gpu_encode(w: torch.Tensor, gs: int):
    packed, scales = ops.encode(w.to(DEV), gs)
    torch.cuda.synchronize()
    return packed.cpu().numpy(), _u16(scales)


def _oracle_encode(w: torch.Tensor, gs: int):
    p, s, _ = O.encode(w.float().numpy(), gs)
    return p, s


def _outliers(w: torch.Tensor, g: torch.Generator, frac=1000, sigma=0.16) -> torch.Tensor:
    idx = torch.randperm(w.numel(), generator=g)[: max(1, w.numel() // frac)]
    signs = torch.where(torch.rand(idx.numel(), generator=g) < 0.5, -1.0, 1.0)
    w.view(-1)[idx] = (sigma * signs).to(w.dtype)
    return w


@pytest.mark.parametrize("gs", [16, 32, 48, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_encode_bit_exact_small(gs, dtype):
    g = torch.Generator().manual_seed(gs * 7 + int(dtype.itemsize))
    w = _outliers(torch.randn(96, 256, generator=g) * 0.02, g).to(dtype)
    pg, sg = _gpu_encode(w, gs)
    po, so = _oracle_encode(w, gs)
    assert np.array_equal(sg, so)
    assert np.array_equal(pg, po)


@pytest.mark.parametrize("shape,gs", [((7, 13), 16), ((5, 19), 32), ((3, 40), 48),
                                      ((1, 1), 32), ((33, 17), 64)])
def test_encode_padding_tail(shape, gs):
    # reference tests/test_ojasx_exhaustive.py:301-320 odd shapes; flat zero padding
    g = torch.Generator().manual_seed(sum(shape))
    w = torch.randn(*shape, generator=g)
    pg, sg = _gpu_encode(w, gs)
    po, so = _oracle_encode(w, gs)
    assert pg.size == O.padded(w.numel(), gs) * 3 // 16
    assert np.array_equal(sg, so) and np.array_equal(pg, po)


def test_encode_edge_magnitudes():
    # zero groups (s = 1e-8 -> fp16 0), tiny groups (fp16 subnormal scales),
    # large groups, exact ties (v = +-0.5, +-1.5), signed zeros
    g = torch.Generator().manual_seed(3)
    rows = [
        torch.zeros(64),
        torch.randn(64, generator=g) * 1e-6,
        torch.randn(64, generator=g) * 3e-8,
        torch.randn(64, generator=g) * 100.0,
        torch.full((64,), -0.0),
        torch.tensor([0.5, -0.5, 1.5, -1.5] * 16),
        torch.tensor([1.0, 0.0] * 32),
        torch.randn(64, generator=g).sign(),
    ]
    w = torch.stack(rows)
    for gs in (16, 32, 64):
        pg, sg = _gpu_encode(w, gs)
        po, so = _oracle_encode(w, gs)
        assert np.array_equal(sg, so), gs
        assert np.array_equal(pg, po), gs


def test_encode_minus_zero_quotient():
    # a negative subnormal weight next to a large one: its quotient by the group scale
    # rounds to -0, where the reference's parity fix flips up (alt = +1 for v >= 0)
    # (fp32 only: a half-precision subnormal over a scale fp16 can hold is never -0)
    rows = []
    for tiny, big in ((-1e-45, 12.0), (-3e-45, 12.0), (-3e-45, 100.0), (-1e-45, 0.5)):
        for pos in (0, 5, 8, 31):
            r = torch.zeros(64)
            r[pos] = tiny
            r[(pos + 1) % 64] = big
            rows.append(r)
    w = torch.stack(rows)
    for gs in (16, 32, 64):
        pg, sg = _gpu_encode(w, gs)
        po, so = _oracle_encode(w, gs)
        assert np.array_equal(sg, so), gs
        assert np.array_equal(pg, po), gs


def test_encode_c1_layer_bit_exact():
    # BASELINE C1: W fp32 4096x4096 ~ N(0, 0.02), CPU generator seed 8101, gs 32
    g = torch.Generator().manual_seed(8101)
    w = torch.randn(4096, 4096, generator=g) * 0.02
    pg, sg = _gpu_encode(w, 32)
    po, so = _oracle_encode(w, 32)
    assert np.array_equal(sg, so)
    assert np.array_equal(pg, po)


def test_encode_c4_fp16_layer_with_outliers_bit_exact():
    # BASELINE C4 distribution on the largest layer shape (gate/up 14336x4096)
    g = torch.Generator().manual_seed(9000)
    w = _outliers((torch.randn(14336, 4096, generator=g) * 0.02).half(), g)
    pg, sg = _gpu_encode(w, 32)
    po, so = _oracle_encode(w, 32)
    assert np.array_equal(sg, so)
    assert np.array_equal(pg, po)


def test_encode_on_device_generated_stack_layer_properties():
    # C4 layers are generated on the GPU.  Size-independent checks on a whole
    # 4096x14336 (down_proj) layer: every code is in range; decoding and
    # re-encoding reproduces the codes (decoded rows are scaled lattice points,
    # so their nearest point is themselves); sampled rows match the oracle.
    gen = torch.Generator(device=DEV).manual_seed(9006)
    w = (torch.randn(4096, 14336, generator=gen, device=DEV) * 0.02).half()
    packed, scales = ops.encode(w, 32)
    trip = packed.view(-1, 3).int()
    codes = torch.stack([trip[:, 0] | ((trip[:, 1] & 15) << 8),
                         (trip[:, 1] >> 4) | (trip[:, 2] << 4)], 1)
    assert int(codes.max()) <= 3280 and int(codes.min()) >= 0
    rec = ops.decode(packed, scales, w.numel(), 32, torch.float32)
    p2, _ = ops.encode(rec, 32)
    assert torch.equal(p2, packed)
    row_bytes, row_scales = 14336 * 3 // 16, 14336 // 32
    for r in (0, 1, 777, 4095):
        po, so = _oracle_encode(w[r].cpu().view(1, -1), 32)
        assert np.array_equal(packed[r * row_bytes:(r + 1) * row_bytes].cpu().numpy(), po)
        assert np.array_equal(_u16(scales[r * row_scales:(r + 1) * row_scales]), so)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("numel,gs", [(96 * 256, 32), (7 * 13, 16), (5 * 19, 32), (1000, 64)])
def test_decode_bit_exact(dtype, numel, gs):
    g = torch.Generator().manual_seed(numel)
    w = torch.randn(numel, generator=g) * 0.05
    po, so = _oracle_encode(w, gs)
    dt_code = {torch.float32: O.DT_F32, torch.float16: O.DT_F16, torch.bfloat16: O.DT_BF16}[dtype]
    ref = O.decode(po, so, numel, gs, dt_code)
    out = ops.decode(torch.from_numpy(po).to(DEV),
                     torch.from_numpy(so.view(np.float16).copy()).to(DEV), numel, gs, dtype)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    else:
        assert np.array_equal(_u16(out), ref)


def test_decode_signed_zero_and_zero_scale():
    # coord -1 times a zero scale is -0.0 in the reference (IEEE product)
    # |w| = 1.2e-8: s = 1.2e-8 + 1e-8 rounds to fp16 zero, while v = w / s ~ +-0.55
    # gives +-1 coordinates
    w = torch.zeros(2, 32)
    w[1] = torch.randn(32).sign() * 1.2e-8
    po, so = _oracle_encode(w, 32)
    for dt, code in ((torch.float32, O.DT_F32), (torch.bfloat16, O.DT_BF16), (torch.float16, O.DT_F16)):
        ref = O.decode(po, so, 64, 32, code)
        out = ops.decode(torch.from_numpy(po).to(DEV),
                         torch.from_numpy(so.view(np.float16).copy()).to(DEV), 64, 32, dt)
        got = out.cpu().numpy().view(np.uint32) if dt == torch.float32 else _u16(out)
        exp = ref.view(np.uint32) if dt == torch.float32 else ref
        assert np.array_equal(got, exp)


def test_packer_api_roundtrip_and_reference_invariants():
    # reference tests/test_sub2bit_lattice.py:40-62 on the device path
    torch.manual_seed(99)
    w = torch.randn(64, 128, device=DEV)
    packed, scales, shape = ojasx_amd.TernaryE8LatticePacker.pack(w, group_size=32)
    assert packed.numel() == int(w.numel() * 1.5 / 8) and shape == (64, 128)
    assert packed.device.type == "cuda" and scales.device.type == "cuda"
    rec = ojasx_amd.TernaryE8LatticePacker.unpack(packed, scales, shape)
    assert rec.shape == w.shape and torch.isfinite(rec).all()
    cos = torch.cosine_similarity(w.flatten(), rec.flatten(), dim=0).item()
    assert cos > 0.70
    # idempotence: decoded weights re-encode to the same codes
    p2, s2, _ = ojasx_amd.TernaryE8LatticePacker.pack(rec, group_size=32)
    assert torch.equal(p2, packed)


def test_packer_cpu_tensors_are_packed_on_gpu_and_returned_on_cpu():
    w = torch.randn(16, 64)
    packed, scales, _ = ojasx_amd.TernaryE8LatticePacker.pack(w, group_size=32)
    assert packed.device.type == "cpu"
    po, so = _oracle_encode(w, 32)
    assert np.array_equal(packed.numpy(), po) and np.array_equal(_u16(scales), so)


@pytest.mark.parametrize("use_hadamard", [False, True])
def test_rowwise_packing_is_byte_exact_to_whole_matrix(use_hadamard):
    # reference tests/test_streaming_e8.py:15-39 (ternary row)
    torch.manual_seed(410)
    weight = torch.randn(12, 64, device=DEV)
    src = ojasx_amd.fwht_block32(weight) if use_hadamard else weight
    exp_codes, exp_scales, _ = ojasx_amd.TernaryE8LatticePacker.pack(src, group_size=32)
    codes, scales = ojasx_amd.pack_weight_rowwise(weight, bitrate=1.5, group_size=32, row_block=5,
                                                  use_hadamard=use_hadamard)
    assert torch.equal(codes, exp_codes) and torch.equal(scales, exp_scales)


def test_encode_does_not_call_cpu_on_device_tensors():
    # reference tests/test_device_native_e8_unpacking.py:27-68: no host round trip
    from unittest.mock import patch

    w = torch.randn(64, 64, device=DEV)
    orig = torch.Tensor.cpu

    def forbidden(self, *a, **k):
        if self.is_cuda:
            raise RuntimeError("FORBIDDEN_HOST_DEVICE_TRANSFER")
        return orig(self, *a, **k)

    with patch.object(torch.Tensor, "cpu", forbidden):
        packed, scales, shape = ojasx_amd.TernaryE8LatticePacker.pack(w, group_size=32)
        rec = ojasx_amd.TernaryE8LatticePacker.unpack(packed, scales, shape)
        assert rec.is_cuda


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_negative_zero_of_zero_scales(dtype):
    # arbitrary valid codes with zero scales: coord -1 times scale 0 is -0 in the reference
    # (coords.to(dtype) * scales.to(dtype), lattice.py:414-418)
    rng = np.random.default_rng(77)
    n, gs = 64 * 128, 32
    codes = rng.integers(0, 3281, n // 8)
    c0, c1 = codes[0::2], codes[1::2]
    packed = np.stack([c0 & 0xFF, ((c0 >> 8) & 0xF) | ((c1 & 0xF) << 4), (c1 >> 4) & 0xFF],
                      axis=1).astype(np.uint8).reshape(-1)
    s = (np.abs(rng.standard_normal(n // gs)) * 0.02).astype(np.float16)
    s[::3] = 0
    out = ops.decode(torch.from_numpy(packed).to(DEV), torch.from_numpy(s).to(DEV), n, gs, dtype)
    ref = O.decode(packed, s.view(np.uint16), n, gs,
                   O.DT_F16 if dtype == torch.float16 else O.DT_BF16)
    assert (ref == 0x8000).any()
    assert np.array_equal(_u16(out), ref)
